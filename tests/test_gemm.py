"""GPU parity of the MFMA prefill GEMM through the C-ABI, against the CPU oracle on the same seeded
inputs.

Mirrors the reference's tests/test_kernels.py test_gemm (134-179), test_gemm_splitk (68-131),
test_gemm_int8 (443-470) and test_gemm_graph_after_workspace_growth (182-205): every tile config
(forced through hi_gemm_force_config) and the automatic choice, split-K 2/4/8 at batched-decode M,
short K (one and two K tiles per split), every epilogue, the partial SwiGLU tile with a sentinel
row, int8 weights (the oracle computes on fp16(q * s)), and a captured split-K GEMM replayed after
the workspace grew. Large shapes are checked on sampled rows (rows are computed independently, so
the oracle's GEMM of those rows is the exact reference for them). Adds bitwise determinism of
split-K (partials are summed in split order whatever the arrival order), and the batched-decode
tiles (M <= 64, deep rings; the role of the reference's skinny kernel, kernels.cuh:896-1115) at
every M class, epilogue, weight format and split count, including a K tail of 32, a half-filled
last column tile, and graph replays, and split-K GEMMs issued from two host threads at once.
"""
import numpy as np
import pytest

from tests._util import bits, check, cuda, gpu, h16, host, interleave, rng

pytestmark = gpu


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


def sample_rows(M, r, n=24):
    if M <= n:
        return np.arange(M)
    return np.unique(np.concatenate([[0, M - 1], r.choice(M, n - 2, replace=False)]))


def gemm_check(hi, O, name, A, W, r, epi=0, bias=None, scales=None, res=None, tol=(3e-3, 3e-3)):
    """Run the GPU GEMM on the full shape; compare sampled rows with the oracle."""
    import torch
    M = A.shape[0]
    out = cuda(res) if res is not None else None
    got = host(hi.gemm(cuda(A), cuda(W), out=out, epi=epi, bias=None if bias is None else cuda(bias),
                       scales=None if scales is None else cuda(scales)))
    rows = sample_rows(M, r)
    ref = O.gemm(np.ascontiguousarray(A[rows]), W, out=None if res is None else np.ascontiguousarray(res[rows]),
                 epi=epi, bias=bias, scales=scales)
    check(name, got[rows], ref, *tol)
    torch.cuda.synchronize()


# The library's tile-config count. Not read from the library at collection time: libhipinfer.so must
# be loaded after torch has initialised its HIP runtime. test_config_count_is_current keeps it honest.
NUM_CFGS = 20
# every tile configuration, and the automatic choice (-1)
CFGS = list(range(-1, NUM_CFGS))


def test_config_count_is_current(hi):
    assert hi.lib.hi_gemm_num_configs() == NUM_CFGS, "update NUM_CFGS: every config must be tested"


def need_cfg(hi, cfg):
    if cfg >= hi.lib.hi_gemm_num_configs():
        pytest.skip(f"the library has {hi.lib.hi_gemm_num_configs()} configs")


def last_choice(hi):
    import ctypes
    c, sp = ctypes.c_int(), ctypes.c_int()
    hi.lib.hi_gemm_last_choice(ctypes.byref(c), ctypes.byref(sp))
    return c.value, sp.value


def cfg_shape(hi, cfg):
    """(bm, bn, bk, waves per K group, K groups) of a tile config, from hi_gemm_config_desc."""
    import ctypes
    import re
    buf = ctypes.create_string_buffer(128)
    hi.lib.hi_gemm_config_desc(cfg, buf, 128)
    m = re.search(r"(\d+)x(\d+)x(\d+) waves (\d+)x(\d+)x(\d+)", buf.value.decode())
    return int(m[1]), int(m[2]), int(m[3]), int(m[4]) * int(m[5]), int(m[6])


def cfg_runs(hi, cfg, q8, K):
    """Whether a forced config runs for this weight format and K, by the library's documented rule:
    every wave issues whole 1 KB DMA instructions per K tile for the A tile and the W tile (int8 W rows
    are half as wide), and the 128-deep tiles take fp16 weights with K % 128 == 0; otherwise the
    automatic choice runs instead."""
    bm, bn, bk, nw, kg = cfg_shape(hi, cfg)
    a, b = bm * 2 * bk, bn * (bk if q8 else 2 * bk)
    ok = a % (1024 * nw) == 0 and b % (1024 * nw) == 0 and a >= 1024 * nw and b >= 1024 * nw
    # K groups split the K tiles evenly inside the block: K a whole number of tiles, per group too
    return ok and (bk < 128 or (not q8 and K % 128 == 0)) and (kg == 1 or (K % bk == 0 and (K // bk) % kg == 0))


def assert_ran(hi, cfg, q8, K, what):
    """The last launch ran the forced config when it can run, and something else when it cannot."""
    if cfg < 0:
        return
    got = last_choice(hi)[0]
    if cfg_runs(hi, cfg, q8, K):
        assert got == cfg, f"{what}: forced config {cfg} did not run (ran {got})"
    else:
        assert got != cfg, f"{what}: config {cfg} ran where it does not fit"


SHAPES = [(128, 2560, 2048), (77, 2048, 5632), (512, 32000, 2048), (1000, 2048, 2048), (300, 1152, 896),
          (64, 6144, 4096), (257, 4096, 14336)]


@pytest.mark.parametrize("cfg", CFGS)
def test_gemm_configs(hi, O, cfg):
    need_cfg(hi, cfg)
    r = rng(300 + cfg)
    hi.lib.hi_gemm_force_config(cfg)
    try:
        for M, N, K in SHAPES:
            A = h16(r, M, K)
            W = h16(r, N, K, sd=0.02)
            gemm_check(hi, O, f"gemm cfg={cfg} M={M} N={N} K={K}", A, W, r)
            assert_ran(hi, cfg, False, K, f"M={M} N={N} K={K}")
        M, H, I = 200, 2048, 5632
        A = h16(r, M, H)
        W = h16(r, 1152, H, sd=0.02)
        b = h16(r, 1152)
        gemm_check(hi, O, f"gemm+bias cfg={cfg}", A, W, r, bias=b)
        gu = interleave(h16(r, I, H, sd=0.02), h16(r, I, H, sd=0.02))
        gemm_check(hi, O, f"gemm+swiglu cfg={cfg}", A, gu, r, epi=2, tol=(4e-3, 4e-3))
        res = h16(r, M, H)
        a = h16(r, M, I)
        W2 = h16(r, H, I, sd=0.02)
        gemm_check(hi, O, f"gemm+residual cfg={cfg}", a, W2, r, epi=1, res=res, tol=(4e-3, 2e-3))
        assert_ran(hi, cfg, False, I, "residual")
        # SwiGLU with a partial last column tile: nothing may be written past column I2
        I2 = 608
        gu2 = interleave(h16(r, I2, H, sd=0.02), h16(r, I2, H, sd=0.02))
        buf = np.full((M + 1, I2), 7.0, np.float16)
        bd = cuda(buf)
        hi.gemm(cuda(A), cuda(gu2), out=bd[:M], epi=2)
        got = host(bd)
        check(f"gemm+swiglu cfg={cfg} I={I2} (partial tile)", got[:M], O.gemm(A, gu2, epi=2), 4e-3, 4e-3)
        assert (got[M] == 7.0).all(), "wrote past the output"
    finally:
        hi.lib.hi_gemm_force_config(-1)


@pytest.mark.parametrize("cfg", CFGS)
def test_gemm_writes_nothing_past_n(hi, O, cfg):
    """N % 32 == 16 (allowed: N % 16 == 0): the last 32-column MFMA tile ends 16 columns past N.
    With padded rows (ldc = N + 16) the padding and a sentinel row past M must keep their values,
    for the store, bias and residual epilogues, one split and four."""
    need_cfg(hi, cfg)
    r = rng(370 + cfg)
    hi.lib.hi_gemm_force_config(cfg)
    try:
        for M, N, K, epi, sp in [(5, 1552, 992, 0, 1), (70, 1040, 1024, 1, 1), (33, 1552, 1024, 0, 4),
                                 (5, 528, 2048, 1, 4), (130, 1040, 1536, 0, 1), (40, 528, 1024, 1, 3)]:
            hi.lib.hi_gemm_force_splits(sp)
            A = h16(r, M, K)
            W = h16(r, N, K, sd=0.02)
            b = h16(r, N) if epi == 0 else None
            buf = np.full((M + 1, N + 16), 7.0, np.float16)
            res = h16(r, M, N)
            if epi == 1:
                buf[:M, :N] = res
            bd = cuda(buf)
            hi.gemm(cuda(A), cuda(W), out=bd[:M, :N], epi=epi, bias=None if b is None else cuda(b))
            got = host(bd)
            ref = O.gemm(A, W, epi=epi, bias=b, out=res.copy() if epi == 1 else None)
            check(f"cfg={cfg} M={M} N={N} epi={epi} split={sp}", got[:M, :N], ref, 4e-3, 3e-3)
            assert_ran(hi, cfg, False, K, f"M={M} N={N} K={K}")
            assert (got[:, N:] == 7.0).all() and (got[M] == 7.0).all(), f"cfg={cfg} N={N}: wrote past column N or row M"
    finally:
        hi.lib.hi_gemm_force_config(-1)
        hi.lib.hi_gemm_force_splits(-1)


def wide_wave_cfgs(hi):
    """Configs whose waves each span the tile's full width (waves WM x 1, one K group): the tiles
    whose epilogue goes through LDS when C rows are 16-byte addressable."""
    import ctypes
    import re
    out = []
    for cfg in range(hi.lib.hi_gemm_num_configs()):
        buf = ctypes.create_string_buffer(128)
        hi.lib.hi_gemm_config_desc(cfg, buf, 128)
        m = re.search(r"waves (\d+)x(\d+)x(\d+)", buf.value.decode())
        if int(m[2]) == 1 and int(m[3]) == 1:
            out.append(cfg)
    return out


@pytest.mark.parametrize("epi", [0, 1, 2])
def test_gemm_staged_epilogue_matches_direct(hi, O, epi):
    """The staged epilogue (C rows 16-byte addressable) and the direct one (ldc % 8 == 4: 8-byte
    stores only) give the same bits on the tiles that have both, with a partial row tile (M = 200),
    a last column tile that ends 16 columns past N (N % 32 == 16; SwiGLU N % 32 == 0), a bias, and
    the residual; the row padding is left alone by both."""
    import torch
    cfgs = wide_wave_cfgs(hi)
    assert cfgs, "no wide-wave tile config"
    r = rng(390 + epi)
    M, K = 200, 1024
    N = 1056 if epi == 2 else 1040
    n_out = N // 2 if epi == 2 else N
    A = h16(r, M, K)
    W = interleave(h16(r, N // 2, K, sd=0.02), h16(r, N // 2, K, sd=0.02)) if epi == 2 else h16(r, N, K, sd=0.02)
    b = h16(r, N) if epi == 0 else None
    res = h16(r, M, n_out)
    ref = O.gemm(A, W, epi=epi, bias=b, out=res.copy() if epi == 1 else None)
    for cfg in cfgs:
        hi.lib.hi_gemm_force_config(cfg)
        hi.lib.hi_gemm_force_splits(1)
        try:
            outs = []
            for pad in (0, 4):  # ldc = n_out (staged), n_out + 4 (direct)
                buf = np.full((M, n_out + pad), 7.0, np.float16)
                if epi == 1:
                    buf[:, :n_out] = res
                bd = cuda(buf)
                hi.gemm(cuda(A), cuda(W), out=bd[:, :n_out], epi=epi, bias=None if b is None else cuda(b))
                got = host(bd)
                assert last_choice(hi)[0] == cfg
                assert (got[:, n_out:] == 7.0).all(), f"cfg={cfg} pad={pad}: wrote into the row padding"
                check(f"cfg={cfg} epi={epi} ldc={n_out + pad}", got[:, :n_out], ref, 4e-3, 4e-3)
                outs.append(got[:, :n_out])
            assert np.array_equal(bits(outs[0]), bits(outs[1])), f"cfg={cfg} epi={epi}: staged and direct differ"
        finally:
            hi.lib.hi_gemm_force_config(-1)
            hi.lib.hi_gemm_force_splits(-1)
            torch.cuda.synchronize()


def test_gemm_large_prefill_shapes(hi, O):
    """Llama-3.2-3B prefill shapes at M = 2000 (non-tile-multiple), automatic choice."""
    r = rng(310)
    for N, K in [(5120, 3072), (3072, 8192), (16384, 3072)]:
        A = h16(r, 2000, K)
        W = h16(r, N, K, sd=0.02)
        gemm_check(hi, O, f"gemm M=2000 N={N} K={K}", A, W, r)


@pytest.mark.parametrize("sp", [2, 4, 8])
def test_gemm_splitk(hi, O, sp):
    r = rng(320 + sp)
    H, I = 2048, 5632
    hi.lib.hi_gemm_force_splits(sp)
    try:
        for M in [9, 32, 64]:
            x = h16(r, M, H)
            W = h16(r, 2560, H, sd=0.02)
            gemm_check(hi, O, f"split={sp} M={M}", x, W, r)
            b = h16(r, 2560)
            gemm_check(hi, O, f"split={sp} +bias M={M}", x, W, r, bias=b)
            res = h16(r, M, H)
            a = h16(r, M, I)
            W2 = h16(r, H, I, sd=0.02)
            gemm_check(hi, O, f"split={sp} +residual M={M}", a, W2, r, epi=1, res=res, tol=(4e-3, 2e-3))
            gu = interleave(h16(r, I, H, sd=0.02), h16(r, I, H, sd=0.02))
            gemm_check(hi, O, f"split={sp} +swiglu M={M}", x, gu, r, epi=2, tol=(4e-3, 4e-3))
    finally:
        hi.lib.hi_gemm_force_splits(-1)


def test_gemm_short_k(hi, O):
    """One and two K tiles per split (K % 32 is the floor); a split that does not divide the K
    tiles leaves no empty split."""
    r = rng(330)
    try:
        for cfg in CFGS:
            hi.lib.hi_gemm_force_config(cfg)
            for sp in [1, 2]:
                hi.lib.hi_gemm_force_splits(sp)
                for M, K in [(300, 32 * sp), (300, 64 * sp), (129, 96), (33, 32), (300, 128 * sp), (70, 384)]:
                    x = h16(r, M, K)
                    W = h16(r, 1024, K, sd=0.02)
                    gemm_check(hi, O, f"short-K cfg={cfg} split={sp} M={M} K={K}", x, W, r)
                    assert_ran(hi, cfg, False, K, f"short-K split={sp} M={M} K={K}")
    finally:
        hi.lib.hi_gemm_force_config(-1)
        hi.lib.hi_gemm_force_splits(-1)


@pytest.mark.parametrize("cfg", CFGS)
def test_gemm_int8(hi, O, cfg):
    need_cfg(hi, cfg)
    r = rng(340 + cfg)
    H, I = 2048, 5632
    hi.lib.hi_gemm_force_config(cfg)
    try:
        for M, N, K in [(128, 2560, 2048), (77, 2048, 5632), (300, 1152, 896), (2000, 3072, 8192), (9, 2560, 2048)]:
            q, s = O.quantize_rows(h16(r, N, K, sd=0.02))
            A = h16(r, M, K)
            gemm_check(hi, O, f"int8 cfg={cfg} M={M} N={N} K={K}", A, q, r, scales=s)
            assert_ran(hi, cfg, True, K, f"int8 M={M} N={N} K={K}")
        M = 200
        A = h16(r, M, H)
        q, s = O.quantize_rows(h16(r, 2560, H, sd=0.02))
        b = h16(r, 2560)
        gemm_check(hi, O, f"int8+bias cfg={cfg}", A, q, r, bias=b, scales=s)
        qg, sg = O.quantize_rows(interleave(h16(r, I, H, sd=0.02), h16(r, I, H, sd=0.02)))
        gemm_check(hi, O, f"int8+swiglu cfg={cfg}", A, qg, r, epi=2, scales=sg, tol=(4e-3, 4e-3))
        qd, sd = O.quantize_rows(h16(r, H, I, sd=0.02))
        gemm_check(hi, O, f"int8+residual cfg={cfg}", h16(r, M, I), qd, r, epi=1, scales=sd, res=h16(r, M, H),
                   tol=(4e-3, 2e-3))
    finally:
        hi.lib.hi_gemm_force_config(-1)
    for sp in [2, 4]:
        hi.lib.hi_gemm_force_splits(sp)
        try:
            for M in [9, 64]:
                q, s = O.quantize_rows(h16(r, 2560, H, sd=0.02))
                gemm_check(hi, O, f"int8 split={sp} M={M}", h16(r, M, H), q, r, bias=h16(r, 2560), scales=s)
        finally:
            hi.lib.hi_gemm_force_splits(-1)


def test_gemm_splitk_deterministic(hi):
    r = rng(350)
    A = cuda(h16(r, 64, 4096))
    W = cuda(h16(r, 3072, 4096, sd=0.02))
    hi.lib.hi_gemm_force_splits(8)
    try:
        a = host(hi.gemm(A, W))
        for _ in range(3):
            assert np.array_equal(bits(host(hi.gemm(A, W))), bits(a))
    finally:
        hi.lib.hi_gemm_force_splits(-1)


def test_gemm_graph_after_workspace_growth(hi, O):
    """A split-K GEMM captured in a graph keeps the workspace it was captured with: a later, larger
    split-K GEMM must not free it. The graph is replayed several times with eager work between the
    replays, and every replay is checked."""
    import torch
    r = rng(360)
    H = 2048
    hi.lib.hi_gemm_force_splits(4)
    try:
        xh = h16(r, 16, H)
        Wh = h16(r, 2560, H, sd=0.02)
        x, W = cuda(xh), cuda(Wh)
        out = torch.empty(16, 2560, dtype=torch.float16, device="cuda")
        hi.gemm(x, W, out=out)  # eager: sizes the workspace
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            hi.gemm(x, W, out=out)
        A = cuda(h16(r, 1024, H))
        W2 = cuda(h16(r, 8192, H, sd=0.02))
        hi.gemm(A, W2)  # outgrows the workspace
        del A, W2
        junk = torch.full((32 << 20,), 1e4, device="cuda")  # may land on a freed workspace
        ref = O.gemm(xh, Wh)
        for _ in range(3):
            out.zero_()
            g.replay()
            torch.cuda.synchronize()
            check("split-K graph replay after workspace growth", host(out), ref, 3e-3, 3e-3)
            hi.gemm(x, W)  # eager split-K work between replays
            torch.cuda.synchronize()
        del junk
    finally:
        hi.lib.hi_gemm_force_splits(-1)


SMALL_M = [3, 5, 6, 15]
# (M, N, K, epi, splits): M classes 1..32 and 33..64, K tails of 32 (K = 992, 1504), a last column
# tile partly past N, SwiGLU
SKINNY_CASES = [(1, 2048, 1024, 0, 1), (9, 1536, 2048, 1, 2), (16, 2560, 2048, 2, 4), (17, 4096, 1024, 0, 8),
                (32, 1024, 4096, 2, 2), (33, 2048, 1504, 1, 1), (50, 1024, 3072, 0, 4), (64, 4096, 1024, 2, 8),
                (64, 1552, 992, 1, 2), (5, 1552, 992, 0, 8), (64, 512, 256, 0, 1)]


@pytest.mark.parametrize("q8", [False, True], ids=["fp16", "int8"])
@pytest.mark.parametrize("cfg", SMALL_M)
def test_gemm_small_m(hi, O, cfg, q8):
    need_cfg(hi, cfg)
    r = rng(900 + cfg + 10 * q8)
    hi.lib.hi_gemm_force_config(cfg)
    try:
        for M, N, K, epi, sp in SKINNY_CASES:
            hi.lib.hi_gemm_force_splits(sp)
            A = h16(r, M, K)
            W = h16(r, N, K, sd=0.02) if epi != 2 else interleave(h16(r, N // 2, K, sd=0.02), h16(r, N // 2, K, sd=0.02))
            q, s = O.quantize_rows(W) if q8 else (W, None)
            bias = h16(r, N) if epi == 0 and M % 2 else None
            res = h16(r, M, N) if epi == 1 else None
            tol = (4e-3, 4e-3) if epi == 2 else (4e-3, 2e-3) if epi == 1 else (3e-3, 3e-3)
            gemm_check(hi, O, f"small-M cfg={cfg} {'int8' if q8 else 'fp16'} M={M} N={N} K={K} epi={epi} split={sp}",
                       A, q, r, epi=epi, bias=bias, scales=s, res=res, tol=tol)
    finally:
        hi.lib.hi_gemm_force_config(-1)
        hi.lib.hi_gemm_force_splits(-1)


def test_gemm_small_m_deterministic_and_graph(hi, O):
    """Splits summed in split order: bit-identical across runs; a captured split launch replays
    correctly, with eager split launches of another shape between the replays."""
    import torch
    r = rng(950)
    hi.lib.hi_gemm_force_config(6)
    hi.lib.hi_gemm_force_splits(8)
    try:
        xh, Wh = h16(r, 40, 4096), h16(r, 3072, 4096, sd=0.02)
        x, W = cuda(xh), cuda(Wh)
        a = host(hi.gemm(x, W))
        for _ in range(3):
            assert np.array_equal(bits(host(hi.gemm(x, W))), bits(a))
        check("small-M split 8", a, O.gemm(xh, Wh), 3e-3, 3e-3)
        out = torch.empty(40, 3072, dtype=torch.float16, device="cuda")
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            hi.gemm(x, W, out=out)
        x2h, W2h = h16(r, 7, 2048), h16(r, 6144, 2048, sd=0.02)
        x2, W2 = cuda(x2h), cuda(W2h)
        ref2 = O.gemm(x2h, W2h)
        for _ in range(3):
            out.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(bits(host(out)), bits(a)), "graph replay differs from the eager result"
            check("small-M eager between replays", host(hi.gemm(x2, W2)), ref2, 3e-3, 3e-3)
    finally:
        hi.lib.hi_gemm_force_config(-1)
        hi.lib.hi_gemm_force_splits(-1)


def test_gemm_split_k_from_two_threads(hi):
    """Split-K partials live in a workspace per host thread and device (as the reference's
    thread_local one, api.cu:54-73): two host threads issuing split-K GEMMs on their own streams at
    the same time each get the bits of the same GEMM run alone."""
    import threading
    import torch
    r = rng(970)
    hi.lib.hi_gemm_force_config(6)
    hi.lib.hi_gemm_force_splits(8)
    try:
        xs = [cuda(h16(r, 40, 4096)) for _ in range(2)]
        Ws = [cuda(h16(r, 3072, 4096, sd=0.02)) for _ in range(2)]
        ref = [host(hi.gemm(xs[i], Ws[i])) for i in range(2)]
        reps = 16
        outs, errs = [None, None], []
        start = threading.Barrier(2)

        def run(i):
            try:
                s = torch.cuda.Stream()
                with torch.cuda.stream(s):
                    o = [torch.empty(40, 3072, dtype=torch.float16, device="cuda") for _ in range(reps)]
                    start.wait(timeout=120)
                    for k in range(reps):
                        hi.gemm(xs[i], Ws[i], out=o[k])
                s.synchronize()
                outs[i] = [host(t) for t in o]
            except Exception as e:  # reported by the main thread
                errs.append(e)

        th = [threading.Thread(target=run, args=(i,)) for i in range(2)]
        for t in th:
            t.start()
        for t in th:
            t.join()
        assert not errs, errs
        for i in range(2):
            for k in range(reps):
                assert np.array_equal(bits(outs[i][k]), bits(ref[i])), f"thread {i} launch {k}"
    finally:
        hi.lib.hi_gemm_force_config(-1)
        hi.lib.hi_gemm_force_splits(-1)


def test_gemm_small_m_automatic(hi, O):
    """The automatic choice at decode batch sizes (Llama-3.1-8B projections)."""
    r = rng(960)
    for M in [9, 24, 40, 64]:
        for N, K, epi in [(6144, 4096, 0), (4096, 4096, 1), (28672, 4096, 2), (4096, 14336, 1)]:
            A = h16(r, M, K)
            W = h16(r, N, K, sd=0.02)
            res = h16(r, M, N) if epi == 1 else None
            gemm_check(hi, O, f"auto M={M} N={N} K={K} epi={epi}", A, W, r, epi=epi, res=res,
                       tol=(4e-3, 4e-3) if epi == 2 else (4e-3, 2e-3))


def test_gemm_rejects_bad_shapes(hi):
    import torch
    A = torch.zeros(4, 48, dtype=torch.float16, device="cuda")
    W = torch.zeros(64, 48, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        hi.gemm(A, W)  # K % 32 != 0
    A = torch.zeros(4, 64, dtype=torch.float16, device="cuda")
    W = torch.zeros(40, 64, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        hi.gemm(A, W)  # N % 16 != 0
    W = torch.zeros(48, 64, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        hi.gemm(A, W, epi=2)  # SwiGLU needs N % 32 == 0


# the 128-deep tiles and their 64-deep twins: (deep, twin)
DEEP_TWINS = [(17, 3), (18, 7)]


@pytest.mark.parametrize("deep,twin", DEEP_TWINS)
def test_gemm_deep_k_tiles_bit_identical(hi, O, deep, twin):
    """A 128-deep K tile sums its k range in the order of two consecutive 64-deep tiles, so at one
    split the 128-deep config gives the bits of its 64-deep twin (same BM x BN and waves), for every
    epilogue. With 3 splits the split boundaries differ (K tiles of 128 against 64), so there the
    sums are only checked against the oracle."""
    need_cfg(hi, deep)
    assert cfg_shape(hi, deep)[:2] == cfg_shape(hi, twin)[:2] and cfg_shape(hi, deep)[2] == 128
    r = rng(380 + deep)
    H, I = 3072, 8192
    cases = [("store", h16(r, 128, H), h16(r, 5120, H, sd=0.02), 0, h16(r, 5120), None),
             ("residual", h16(r, 100, I), h16(r, H, I, sd=0.02), 1, None, h16(r, 100, H)),
             ("swiglu", h16(r, 77, H), interleave(h16(r, 1024, H, sd=0.02), h16(r, 1024, H, sd=0.02)), 2, None, None),
             ("store K=1152", h16(r, 33, 1152), h16(r, 2048, 1152, sd=0.02), 0, None, None)]
    try:
        for name, A, W, epi, bias, res in cases:
            outs = []
            for c in (deep, twin):
                hi.lib.hi_gemm_force_config(c)
                hi.lib.hi_gemm_force_splits(1)
                o = cuda(res) if res is not None else None
                outs.append(host(hi.gemm(cuda(A), cuda(W), out=o, epi=epi, bias=None if bias is None else cuda(bias))))
                assert last_choice(hi) == (c, 1), f"{name}: config {c} split 1 did not run"
            assert np.array_equal(bits(outs[0]), bits(outs[1])), f"{name}: config {deep} differs from {twin}"
            ref = O.gemm(A, W, epi=epi, bias=bias, out=None if res is None else res.copy())
            check(f"deep cfg={deep} {name}", outs[0], ref, 4e-3, 3e-3)
        # three splits over K = 2048 (16 deep tiles -> 6 + 6 + 4; the twin would split 32 tiles 11 + 11 + 10)
        hi.lib.hi_gemm_force_config(deep)
        hi.lib.hi_gemm_force_splits(3)
        for M, N, epi in [(64, 2560, 0), (128, 3072, 1), (40, 4096, 2)]:
            A = h16(r, M, 2048)
            W = h16(r, N, 2048, sd=0.02) if epi != 2 else interleave(h16(r, N // 2, 2048, sd=0.02),
                                                                     h16(r, N // 2, 2048, sd=0.02))
            res = h16(r, M, N) if epi == 1 else None
            gemm_check(hi, O, f"deep cfg={deep} split=3 M={M} N={N} epi={epi}", A, W, r, epi=epi, res=res,
                       tol=(4e-3, 4e-3) if epi == 2 else (4e-3, 2e-3))
            assert last_choice(hi) == (deep, 3), f"config {deep} split 3 did not run"
    finally:
        hi.lib.hi_gemm_force_config(-1)
        hi.lib.hi_gemm_force_splits(-1)


@pytest.mark.parametrize("M", [128, 512, 1024])
@pytest.mark.parametrize("q8", [False, True], ids=["fp16", "int8"])
def test_gemm_llama32_3b_layer(hi, O, M, q8):
    """C3 (Llama-3.2-3B prefill) at the benchmarked M with the automatic (tuned) choice: QKV
    3072 -> 5120 (store), o 3072 -> 3072 (+ residual), gate/up 3072 -> 2 x 8192 (SwiGLU), down
    8192 -> 3072 (+ residual), fp16 and int8 weights; sampled rows against the oracle."""
    r = rng(400 + M + q8)
    H, I, QKV = 3072, 8192, 5120
    for name, N, K, epi in [("qkv", QKV, H, 0), ("o", H, H, 1), ("gate/up", 2 * I, H, 2), ("down", H, I, 1)]:
        A = h16(r, M, K)
        W = h16(r, N, K, sd=0.02) if epi != 2 else interleave(h16(r, I, H, sd=0.02), h16(r, I, H, sd=0.02))
        s = None
        if q8:
            W, s = O.quantize_rows(W)
        res = h16(r, M, N) if epi == 1 else None
        tol = (4e-3, 4e-3) if epi == 2 else (4e-3, 2e-3) if epi == 1 else (3e-3, 3e-3)
        gemm_check(hi, O, f"C3 {name} {'int8' if q8 else 'fp16'} M={M}", A, W, r, epi=epi, scales=s, res=res, tol=tol)
        c, sp = last_choice(hi)
        assert 0 <= c < NUM_CFGS and sp >= 1, (name, c, sp)


@pytest.mark.parametrize("q8", [False, True], ids=["fp16", "int8"])
def test_gemm_residual_rmsnorm_bit_identical(hi, O, q8):
    """hi_gemm_residual_rmsnorm gives the bits of hi_gemm (epilogue 1) followed by hi_rmsnorm, for
    the new residual stream and its norm alike: on split-K launches (the norm inside the split-K
    second pass), unsplit ones and the automatic choice, at a short M, and for rows wider than
    the fused pass takes (N = 8704 > 8192: the separate norm). Sampled rows against the oracle."""
    import torch
    r = rng(520 + q8)
    try:
        for M, N, K in [(96, 4096, 1024), (300, 2048, 1536), (7, 1024, 512), (64, 8704, 512)]:
            A, x0 = h16(r, M, K), h16(r, M, N)
            W = h16(r, N, K, sd=0.02)
            nw = (r.random(N) + 0.5).astype(np.float16)
            s = None
            if q8:
                W, s = O.quantize_rows(W)
            Ad, Wd, nd = cuda(A), cuda(W), cuda(nw)
            sd = None if s is None else cuda(s)
            for sp in (-1, 1, 2, 3):
                # the fused call first (automatic: its own tuning, which times the norm too), then
                # the two calls forced onto the tile and split count it ran
                hi.lib.hi_gemm_force_config(-1)
                hi.lib.hi_gemm_force_splits(sp)
                xb = cuda(x0)
                yb = hi.gemm_rmsnorm(Ad, Wd, xb, nd, 1e-5, scales=sd)
                ran = last_choice(hi)
                hi.lib.hi_gemm_force_config(ran[0])
                hi.lib.hi_gemm_force_splits(ran[1])
                xa = cuda(x0)
                hi.gemm(Ad, Wd, out=xa, epi=1, scales=sd)
                ya = hi.rmsnorm(xa, nd, 1e-5)
                assert last_choice(hi) == ran, (M, N, K, sp, ran, last_choice(hi))
                if sp > 1:
                    assert ran[1] > 1, f"split {sp} did not run at M={M} N={N} K={K}"
                what = f"M={M} N={N} K={K} splits={sp} ran={ran}"
                assert np.array_equal(bits(host(xa)), bits(host(xb))), f"residual stream differs: {what}"
                assert np.array_equal(bits(host(ya)), bits(host(yb))), f"norm differs: {what}"
            rows = sample_rows(M, r, 8)
            xr = O.gemm(np.ascontiguousarray(A[rows]), W, out=np.ascontiguousarray(x0[rows]), epi=1, scales=s)
            check(f"gemm_rmsnorm vs oracle M={M} N={N}", host(yb)[rows], O.rmsnorm(xr, nw), 4e-3, 4e-3)
            torch.cuda.synchronize()
    finally:
        hi.lib.hi_gemm_force_config(-1)
        hi.lib.hi_gemm_force_splits(-1)
