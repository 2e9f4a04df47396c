"""came_amd: the CAME 8-bit optimizer step for AMD Instinct MI355X (gfx950).

The optimizer classes keep the reference's (tukisuwa/CAME, ``came_pytorch``)
constructor arguments, ``step()`` semantics and state layout; the step itself
runs in ``libcame8.so`` (hand-written HIP kernels behind the C ABI in
``include/came8.h``).
"""
from .optim import CAME8bit, CAME8bit2D, CAME8bitFull, CAME8bitMemory, CAMECUDA  # noqa: F401

__all__ = ["CAME8bit", "CAME8bit2D", "CAME8bitFull", "CAME8bitMemory", "CAMECUDA"]
__version__ = "0.1.0"
