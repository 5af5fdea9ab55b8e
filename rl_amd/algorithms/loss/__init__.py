"""Drop-ins for ``nemo_rl.algorithms.loss`` (ClippedPG loss and its input preparation)."""

from rl_amd.algorithms.loss.interfaces import (  # noqa: F401
    LossFunction,
    LossInputType,
    LossType,
    MetricNormalizer,
)
from rl_amd.algorithms.loss.loss_functions import (  # noqa: F401
    ClippedPGLossConfig,
    ClippedPGLossDataDict,
    ClippedPGLossFn,
)
