"""bmx_qmatmul_affine_noalloc (split-K partials in the library's static
device scratch) against bmx_qmatmul_affine (the same kernels with a
library-allocated buffer): bit-identical outputs on two calls in a row,
the second smaller, through the C ABI.

Each case runs on a stream of its own, created for it, and calls the
allocation-free entry first, before any other library call on that stream:
no per-stream buffer exists yet that it could fall back on (and while it
runs, the library treats any allocation as an error)."""
import ctypes

import numpy as np
import pytest

from _util import torch_bf16_bits

pytestmark = pytest.mark.gpu


def _call(gpu, name, x, w, s, b, M, N, K, stream):
    import torch

    y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    gpu.call(name, x.data_ptr(), w.data_ptr(), s.data_ptr(), b.data_ptr(), y.data_ptr(), M, N, K, 1, 64, 4,
             ctypes.c_void_p(stream.cuda_stream))
    return y


@pytest.mark.parametrize("shapes", [
    # split-K GEMMs (small tile grids), the second call smaller
    [(64, 1024, 2560), (24, 768, 2048)],
    # a longer K, then a much smaller product
    [(16, 2048, 4096), (12, 512, 1024)],
    # the matrix-core GEMV of up to 8 rows, K split over workgroups (N and K
    # at least 5120, K >= 8192, >= 2^25 weights), then a smaller split GEMV
    [(5, 5120, 25600), (2, 5120, 8192)],
])
def test_noalloc_matches_qmatmul(gpu, shapes):
    import torch

    lib = gpu.load()
    for i, (M, N, K) in enumerate(shapes):
        print(f"noalloc case M={M} N={N} K={K}", flush=True)
        need = lib.bmx_qmatmul_workspace_bytes(M, N, K)
        assert 0 < need <= 16 << 20, need
        w, s, b = gpu.init_qlinear(300 + i, N, K)
        x = gpu.fill_normal_bf16(400 + i, (M, K))
        torch.cuda.synchronize()
        st = torch.cuda.Stream()
        got = _call(gpu, "bmx_qmatmul_affine_noalloc", x, w, s, b, M, N, K, st)
        ref = _call(gpu, "bmx_qmatmul_affine", x, w, s, b, M, N, K, st)
        st.synchronize()
        np.testing.assert_array_equal(torch_bf16_bits(got), torch_bf16_bits(ref))


def test_noalloc_rejects_shapes_beyond_its_scratch(gpu):
    """A shape whose split-K partials exceed the 16 MiB scratch is refused
    before anything is enqueued (the pointers below are never read)."""
    lib = gpu.load()
    M, N, K = 128, 16384, 4096  # 4 splits of 128 x 16384 fp32 partials: 32 MiB
    need = lib.bmx_qmatmul_workspace_bytes(M, N, K)
    if need <= 16 << 20:
        pytest.skip(f"M={M} N={N} K={K} needs only {need} bytes of partials")
    fake = ctypes.c_void_p(0x1000)
    rc = lib.bmx_qmatmul_affine_noalloc(fake, fake, fake, fake, fake, M, N, K, 1, 64, 4, ctypes.c_void_p(0))
    assert rc == gpu.BMX_E_SHAPE and "16777216" in gpu.last_error()
