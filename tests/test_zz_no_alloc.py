"""hi_gemm_noalloc, the GEMM entry point that allocates no device memory (split-K partials in the
library's static scratch, no autotuning), against hi_gemm / hi_gemm_w8 through the C-ABI.

The same (tile, split) gives the same bits on both entry points, so each check forces or reuses one
choice and compares bit for bit; two calls in a row, the second on a smaller problem, show that the
scratch's leftover contents from the first call never reach the second. Also: a forced split whose
partials exceed the scratch is rejected, the automatic choice lowers its split instead, and a
captured graph of the call replays correctly with eager work between the replays.
"""
import numpy as np
import pytest

from tests._util import bits, check, cuda, gpu, h16, host, rng

pytestmark = gpu

SCRATCH_BYTES = 64 << 20


@pytest.fixture(scope="module")
def hi():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from hipinfer_amd import hipinfer
    yield hipinfer
    hipinfer.lib.hi_gemm_force_config(-1)
    hipinfer.lib.hi_gemm_force_splits(-1)


@pytest.fixture(scope="module")
def O():
    from oracle import oracle
    return oracle


def last_choice(hi):
    import ctypes
    c, sp = ctypes.c_int(), ctypes.c_int()
    hi.lib.hi_gemm_last_choice(ctypes.byref(c), ctypes.byref(sp))
    return c.value, sp.value


def problem(r, M, N, K, epi, q8, O):
    A = h16(r, M, K)
    W = h16(r, N, K, sd=0.02)
    s = None
    if q8:
        W, s = O.quantize_rows(W)
    bias = h16(r, N) if epi == 0 else None
    res = h16(r, M, N) if epi == 1 else None
    return A, W, s, bias, res


def run_both(hi, A, W, s, bias, res, epi):
    """(hi_gemm result, its choice), (hi_gemm_noalloc result, its choice) on the same inputs."""
    import torch
    N = W.shape[0]
    Ad, Wd = cuda(A), cuda(W)
    sd = None if s is None else cuda(s)
    bd = None if bias is None else cuda(bias)
    out_a = cuda(res) if res is not None else torch.zeros(A.shape[0], N, dtype=torch.float16, device="cuda")
    out_b = cuda(res) if res is not None else torch.zeros(A.shape[0], N, dtype=torch.float16, device="cuda")
    hi.gemm(Ad, Wd, out=out_a, epi=epi, bias=bd, scales=sd)
    ca = last_choice(hi)
    hi.gemm_noalloc(Ad, Wd, out_b, epi=epi, bias=bd, scales=sd)
    cb = last_choice(hi)
    torch.cuda.synchronize()
    return (host(out_a), ca), (host(out_b), cb)


@pytest.mark.parametrize("q8", [False, True], ids=["fp16", "int8"])
@pytest.mark.parametrize("cfg,sp", [(6, 4), (3, 2), (11, 3), (-1, -1)])
def test_noalloc_matches_gemm_two_calls_second_smaller(hi, O, q8, cfg, sp):
    r = rng(1900 + 10 * cfg + sp + 100 * q8)
    hi.lib.hi_gemm_force_config(cfg)
    hi.lib.hi_gemm_force_splits(sp)
    try:
        for M, N, K, epi in [(64, 4096, 4096, 1), (9, 2560, 2048, 0)]:
            A, W, s, bias, res = problem(r, M, N, K, epi, q8, O)
            (a, ca), (b, cb) = run_both(hi, A, W, s, bias, res, epi)
            assert ca == cb, f"M={M}: the entry points chose {ca} and {cb}"
            if sp > 1:
                assert cb[1] > 1, f"M={M}: the forced split-K did not run ({cb})"
            assert np.array_equal(bits(b), bits(a)), f"M={M} N={N} K={K} cfg={cfg} split={sp}: bits differ"
            ref = O.gemm(A, W, epi=epi, bias=bias, scales=s, out=None if res is None else res.copy())
            check(f"noalloc M={M} N={N} K={K}", b, ref, 4e-3, 3e-3)
    finally:
        hi.lib.hi_gemm_force_config(-1)
        hi.lib.hi_gemm_force_splits(-1)


def test_noalloc_split_limit(hi, O):
    """A forced split whose fp32 partials exceed the static scratch is rejected; the automatic choice
    at the same shape lowers its split to fit and matches the oracle."""
    import torch
    r = rng(1950)
    M, N, K = 512, 16384, 2048
    assert 8 * M * N * 4 > SCRATCH_BYTES
    A = h16(r, M, K)
    W = h16(r, N, K, sd=0.02)
    Ad, Wd = cuda(A), cuda(W)
    out = torch.zeros(M, N, dtype=torch.float16, device="cuda")
    hi.lib.hi_gemm_force_splits(8)
    try:
        with pytest.raises(ValueError):
            hi.gemm_noalloc(Ad, Wd, out)
    finally:
        hi.lib.hi_gemm_force_splits(-1)
    hi.gemm_noalloc(Ad, Wd, out)
    c, sp = last_choice(hi)
    assert sp * M * N * 4 <= SCRATCH_BYTES or sp == 1, (c, sp)
    rows = np.array([0, 7, 100, 311, M - 1])
    check("noalloc auto, large", host(out)[rows], O.gemm(np.ascontiguousarray(A[rows]), W), 3e-3, 3e-3)


def test_noalloc_graph_replay(hi, O):
    """Captured after an eager call (nothing is allocated inside or outside the capture), the split-K
    launch replays to the eager bits, with other eager noalloc calls on the same scratch between
    replays."""
    import torch
    r = rng(1960)
    hi.lib.hi_gemm_force_config(6)
    hi.lib.hi_gemm_force_splits(8)
    try:
        A, W, _, bias, _ = problem(r, 40, 3072, 4096, 0, False, O)
        Ad, Wd, bd = cuda(A), cuda(W), cuda(bias)
        out = torch.zeros(40, 3072, dtype=torch.float16, device="cuda")
        hi.gemm_noalloc(Ad, Wd, out, bias=bd)
        torch.cuda.synchronize()
        eager = host(out).copy()
        check("noalloc eager", eager, O.gemm(A, W, bias=bias), 3e-3, 3e-3)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            hi.gemm_noalloc(Ad, Wd, out, bias=bd)
        A2, W2, _, _, _ = problem(r, 17, 2048, 1024, 1, False, O)
        A2d, W2d = cuda(A2), cuda(W2)
        for _ in range(3):
            out.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(bits(host(out)), bits(eager)), "graph replay differs from the eager call"
            o2 = torch.zeros(17, 2048, dtype=torch.float16, device="cuda")
            hi.gemm_noalloc(A2d, W2d, o2, epi=1)
            torch.cuda.synchronize()
            check("noalloc eager between replays", host(o2), O.gemm(A2, W2, out=np.zeros((17, 2048), np.float16), epi=1),
                  4e-3, 2e-3)
    finally:
        hi.lib.hi_gemm_force_config(-1)
        hi.lib.hi_gemm_force_splits(-1)
