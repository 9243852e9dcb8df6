"""VectorCore tensor/autograd runtime with an MI355X (gfx950) `hip` device.

The module surface is the reference's `vectorcore` Python module
(python/bindings.cpp): ``import vectorcore_amd as vc`` then ``vc.Tensor``,
``vc.Linear``, ``vc.cross_entropy``, ``vc.sgd_step``, ... with ``device="hip"``
accepted wherever a device is. The native extension (and libvc_hip.so, which
it links) must be built in-tree: ``python vectorcore_amd/build.py``.
"""

from ._vectorcore import (  # noqa: F401
    Linear,
    Tensor,
    cross_entropy,
    hip_available,
    hip_defer_products,
    hip_device_name,
    hip_fuse_elementwise,
    hip_gemm_kernel,
    hip_set_gemm_kernel,
    hip_strict_item,
    hip_pool_stats,
    hip_profile,
    hip_profile_read,
    hip_profile_reset,
    log_softmax,
    metal_available,
    metal_device_name,
    metal_gemm_kernel,
    mse_loss,
    sgd_step,
    softmax,
    synchronize,
    zero_grad,
)

DEVICES = ("cpu", "hip")
