"""Numerical constants and enums shared by the attention hot path.

Values mirror mlx_primitives/constants.py of the reference (cited per item)
so that the drop-in keeps the same semantics.
"""

from enum import Enum


class Layout(str, Enum):
    """Tensor layout of attention inputs (mlx_primitives/constants.py:16-28).

    BSHD: (batch, seq, heads, dim); BHSD: (batch, heads, seq, dim). A str enum,
    so ``layout == "BSHD"`` keeps working.
    """

    BSHD = "BSHD"
    BHSD = "BHSD"


# Masked-score value of the tiled/Metal paths (constants.py:100). The GPU
# kernels mask by index arithmetic and never materialise it.
ATTENTION_MASK_VALUE = -1e38

# Largest head dimension of the reference's Metal kernels (constants.py:104);
# the MI355X kernels support the same bound.
METAL_ATTENTION_MAX_HEAD_DIM = 128

# Normaliser epsilon o / (l + eps) of the tiled paths (constants.py:110).
METAL_SOFTMAX_EPSILON = 1e-6

# Dispatch thresholds of flash_attention (constants.py:162-173). The GPU
# kernel serves every size, so these only document the reference behaviour.
FLASH_MAX_SEQ_FOR_REFERENCE = 256
FLASH_SMALL_BATCH_SEQ_THRESHOLD = 512
FLASH_SMALL_BATCH_THRESHOLD = 4
FLASH_MIN_SEQ_FOR_METAL = 64
