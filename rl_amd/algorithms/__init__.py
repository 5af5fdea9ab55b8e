"""Drop-ins for ``nemo_rl.algorithms`` (losses, advantages, sampling filters)."""
