"""ORACLE -- test infrastructure only (see oracle/reference_path.py).

Imported only by tests/, __graft_entry__.smoke() and bench.py's baseline leg, as the
checker and as the timed reference path; never by the card_playing_gym_amd package.
"""
