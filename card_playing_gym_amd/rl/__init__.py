"""Rollout-side device ops (the reference's cardgym.rl helpers that run per wave)."""

from .sampling import masked_probabilities, sample_rows

__all__ = ["masked_probabilities", "sample_rows"]
