"""iris_kernel -- MI355X (gfx950) implementation of Iris-Kernel's compressed
paged KV-cache hot path.

Same import names as the reference package (Hunter2030ZeRo/Iris-Kernel,
src/iris_kernel): ``iris_kernel.fused_kv.fused_rope_int4_paged_append`` and
``iris_kernel.fused_attention.fused_int4_paged_decode_attention``, backed by
hand-written HIP kernels in ``libiris_hip.so`` (C ABI: include/iris_hip.h),
and the reference's eager PyTorch modules ``iris_kernel.torch_eager_kv`` and
``iris_kernel.torch_eager_attention`` (plain torch, any device; the fused
path never calls them).
"""

__version__ = "0.1.0"
