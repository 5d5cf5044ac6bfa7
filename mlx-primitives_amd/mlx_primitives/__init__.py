"""mlx_primitives, MI355X edition: the attention hot path of mlx-primitives
(flash / sliding-window / chunked-cross attention forward and paged-KV decode)
on hand-written gfx950 HIP kernels, with the reference's Python API over
PyTorch-ROCm tensors.

Import ``torch`` first (the kernels bind to torch's HIP runtime); the HIP
library is loaded lazily on the first call.
"""

from mlx_primitives.constants import Layout

__version__ = "0.1.0"

__all__ = ["Layout", "__version__"]
