"""rl_amd — MI355X (gfx950) kernels for NeMo-RL's token-logprob and policy-loss hot path.

Subpackages mirror the reference's import paths:

* ``rl_amd.distributed.model_utils``      -> ``nemo_rl.distributed.model_utils``
* ``rl_amd.algorithms.logits_sampling_utils`` -> ``nemo_rl.algorithms.logits_sampling_utils``
* ``rl_amd.algorithms.loss``              -> ``nemo_rl.algorithms.loss``
* ``rl_amd.algorithms.advantage_estimator`` -> ``nemo_rl.algorithms.advantage_estimator``
* ``rl_amd.algorithms.utils``             -> ``nemo_rl.algorithms.utils`` (math helpers)

The compute runs in ``rl_amd/libmirl.so`` (see ``include/mirl.h``); importing
the package does not load it, calling a kernel does.
"""

__version__ = "0.1.0"
