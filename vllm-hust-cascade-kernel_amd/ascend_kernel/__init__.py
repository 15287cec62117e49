"""Import-name alias for drop-in use: ``import ascend_kernel`` (the reference's
package name, ascend-kernel/python/ascend_kernel/ascend_kernel/__init__.py)
registers the same ``torch.ops.npu.*`` ops, here backed by the gfx950 kernels."""
from cascade_amd import *  # noqa: F401,F403
from cascade_amd import ops  # noqa: F401
