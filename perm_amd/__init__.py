"""perm_amd -- MI355X-native encoder hot path of coldpress (asystemoffields/PERM).

Drop-in GPU backend for the reference's encode stage: the same Python API as
``coldpress.kquant`` (QUANTIZE / DEQUANTIZE / roundtrip), ``coldpress.ef``
(cholesky_inv_upper, ef_encode) and the Hessian hook of ``coldpress.hessians``,
executed by hand-written gfx950 HIP kernels in ``libcoldpress_hip.so`` through a
C ABI (include/coldpress_hip.h). PyTorch provides device memory and streams.

There is no CPU fallback: every entry point raises if the HIP library is not
built or no GPU is visible.
"""
__version__ = "0.1.0"
