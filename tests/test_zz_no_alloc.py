"""cssm_proj_in_noalloc (static device scratch, no allocation) against cssm_proj_in
(caller's workspace), both called through the C ABI: identical outputs and ctx on
two calls in a row, the second smaller, for the persistent (K <= 64, one ctx slot
per tile) and the K-chunked (K > 64, tiles spanning frames) kernels; sizes beyond
the scratch are refused before any GPU work."""

import numpy as np
import pytest

from tests.gpu_util import print_case

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cssm_amd import _lib
    return _lib


def _run(lib_mod, entry, x, Wt, b, F, HW, dt_out):
    lib = lib_mod.load()
    K, N = Wt.shape
    lo = torch.empty((F, N // 2, HW), dtype=dt_out, device="cuda")
    hi = torch.empty_like(lo)
    ctx = torch.empty((F, N // 2), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    dts = {torch.float32: lib_mod.F32, torch.bfloat16: lib_mod.BF16}
    args = (x.data_ptr(), dts[x.dtype], F, HW, K, N, Wt.data_ptr(), b.data_ptr(), lo.data_ptr(), hi.data_ptr(),
            dts[dt_out], 1, 1, ctx.data_ptr())
    if entry == "noalloc":
        st = lib.cssm_proj_in_noalloc(*args, stream)
    else:
        nbytes = int(lib.cssm_proj_in_workspace_size(F, HW, K, N))
        ws = torch.empty(max(1, nbytes // 4), dtype=torch.float32, device="cuda")
        st = lib.cssm_proj_in(*args, ws.data_ptr(), nbytes, stream)
    assert st == 0, lib.cssm_last_error()
    torch.cuda.synchronize()
    return lo, hi, ctx


# (F, HW, K, N, in dtype): each pair is two calls in a row, the second with a smaller input
CASES = [
    ((64, 16384, 64, 128, torch.float32), (3, 1024, 64, 128, torch.float32)),     # persistent, C2-shaped frames
    ((40, 196, 224, 448, torch.bfloat16), (6, 49, 224, 448, torch.bfloat16)),     # K-chunked, tiles span frames
]


@pytest.mark.parametrize("pair", CASES, ids=["persistent", "k_chunked"])
def test_noalloc_matches_workspace_entry_point(lib, pair):
    for F, HW, K, N, dt in pair:
        print_case(test="proj_in_noalloc", F=F, HW=HW, K=K, N=N, dtype=str(dt))
        g = torch.Generator(device="cuda").manual_seed(F * 7 + HW)
        x = torch.randn((F * HW, K), generator=g, device="cuda").to(dt)
        Wt = torch.randn((K, N), generator=g, device="cuda") / np.sqrt(K)
        b = torch.randn((N,), generator=g, device="cuda") * 0.1
        want = _run(lib, "workspace", x, Wt, b, F, HW, torch.float32)
        got = _run(lib, "noalloc", x, Wt, b, F, HW, torch.float32)
        for a, w in zip(got, want):
            assert torch.equal(a, w)


def test_noalloc_without_ctx(lib):
    lib_ = lib.load()
    F, HW, K, N = 2, 1024, 64, 128
    x = torch.randn((F * HW, K), device="cuda")
    Wt = torch.randn((K, N), device="cuda") / 8
    b = torch.zeros(N, device="cuda")
    lo = torch.empty((F, N // 2, HW), device="cuda")
    hi = torch.empty_like(lo)
    stream = torch.cuda.current_stream().cuda_stream
    st = lib_.cssm_proj_in_noalloc(x.data_ptr(), lib.F32, F, HW, K, N, Wt.data_ptr(), b.data_ptr(), lo.data_ptr(),
                                   hi.data_ptr(), lib.F32, 0, 0, None, stream)
    assert st == 0
    torch.cuda.synchronize()
    ref = (x @ Wt + b).view(F, HW, N).transpose(1, 2)
    assert torch.allclose(lo, ref[:, : N // 2], rtol=1e-5, atol=1e-5)
