"""``avey_kernels.ops`` of the reference, served by this build.

Same public entry points, signatures and defaults (``avey_kernels/ops.py:117-147``),
the same input contract (``_validate``, ``ops.py:23-46``) and activation dispatch
(``_activate``, ``ops.py:49-58``). ``_reference`` is the differentiable eager
PyTorch path (``ops.py:61-91``), which this build calls ``_eager``.
"""

from avey_kernel_amd.ops import _activate, _dispatch, _validate, avey, avey_b
from avey_kernel_amd.ops import _eager as _reference

__all__ = ['avey', 'avey_b']
