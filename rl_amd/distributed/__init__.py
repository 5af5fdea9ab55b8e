"""Drop-ins for ``nemo_rl.distributed`` (logprob numerics only)."""
