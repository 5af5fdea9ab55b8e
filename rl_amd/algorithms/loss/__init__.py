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
from rl_amd.algorithms.loss.loss_input import (  # noqa: F401
    prepare_loss_input,
    prepare_packed_loss_input,
)
from rl_amd.algorithms.loss.wrapper import (  # noqa: F401
    SequencePackingFusionLossWrapper,
    SequencePackingLossWrapper,
    wrap_loss_fn_with_input_preparation,
)
