"""Avey and Avey-B contextualizer operations (drop-in for the reference package).

The reference's callers import ``avey`` and ``avey_b`` from ``avey_kernels``
(``avey_kernels/__init__.py:3-5`` of HusamettinYilmazz/avey_kernel). This
package keeps that import path and that module layout; the implementation is
``avey_kernel_amd`` (the fused gfx950 HIP kernels behind ``libavey_hip.so``).
"""

from .ops import avey, avey_b

__all__ = ['avey', 'avey_b']
