"""Game embedders on the device path (the token -> trunk-input side of a rollout step)."""
