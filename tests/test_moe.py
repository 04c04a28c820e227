"""GPU parity of the MoE router and experts through the C-ABI, against the CPU oracle.

Mirrors the reference's tests/test_kernels.py test_moe (473-518): Granite-, Mixtral- and
OLMoE-shaped layers, M in {1, 3, 4, 8, 37, 300}; the router's expert indices and order on rows
without a near-tie among the top k+1 logits, and its weights; the experts through the automatic,
GEMV and grouped paths given the kernel's own routing; the exact-tie known answer (experts 2
and 5 -> [2, 5], weights 1/2). Adds: the grouped path replayed from a captured graph (it never
returns to the host), and expert ids outside [0, E) contributing nothing.
"""
import numpy as np
import pytest

from tests._util import check, cuda, gpu, host, rng

pytestmark = gpu


@pytest.fixture(scope="module")
def hi():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from hipinfer_amd import hipinfer
    return hipinfer


@pytest.fixture(scope="module")
def O():
    from oracle import oracle
    return oracle


def rn(r, *shape, s=1.0):
    return (r.standard_normal(shape) * s).astype(np.float16)


LAYERS = [("granite-like", 32, 8, 1024, 512, 3, 0.22), ("mixtral-like", 8, 2, 512, 1024, 1, 1.0),
          ("olmoe-like", 64, 8, 2048, 1024, 2, 1.0), ("max-k", 128, 16, 512, 256, 1, 1.0),
          ("max-e", 256, 4, 256, 128, 3, 1.0)]


@pytest.mark.parametrize("name,E,k,H,I,flags,scale", LAYERS, ids=[l[0] for l in LAYERS])
def test_moe_router_and_experts(hi, O, name, E, k, H, I, flags, scale):
    r = rng(400 + E)
    Wr = rn(r, E, H, s=0.05)
    wgu, wdn = rn(r, E, 2 * I, H, s=0.02), rn(r, E, H, I, s=0.02)
    Wr_d, wgu_d, wdn_d = cuda(Wr), cuda(wgu), cuda(wdn)
    for M in [1, 3, 4, 8, 37, 300]:
        xn, x = rn(r, M, H), rn(r, M, H)
        idx_d, w_d = hi.moe_router(cuda(xn), Wr_d, k, flags)
        idx, w = host(idx_d), host(w_d)
        ridx, rw = O.moe_router(xn, Wr, k, flags)
        logits = (xn.astype(np.float64) @ Wr.astype(np.float64).T).astype(np.float16).astype(np.float64)
        top = -np.sort(-logits, axis=1)[:, :min(k + 1, E)]
        clear = (top[:, :-1] - top[:, 1:]).min(1) > 1e-2  # rows where summation order cannot flip a pick
        same = (idx == ridx).all(1)
        assert not (clear & ~same).any(), f"{name} M={M}: {(clear & ~same).sum()} clear rows routed differently"
        if same.any():
            check(f"{name} router weights M={M}", w[same], rw[same], 2e-3, 1e-2)
        ref = O.moe_experts(xn, wgu, wdn, idx, w, x.copy(), flags, scale)
        for path in (0, 1, 2):
            out = host(hi.moe_experts(cuda(xn), wgu_d, wdn_d, idx_d, w_d, cuda(x), flags, scale, path))
            check(f"{name} experts M={M} path={['auto', 'gemv', 'grouped'][path]}", out, ref, 4e-3, 4e-3)


def test_moe_router_exact_tie(hi):
    r = rng(410)
    E, k, H = 8, 2, 256
    Wr = rn(r, E, H, s=0.01)
    Wr[2] = Wr[5] = 0.05
    xn = (r.random((4, H)) + 0.5).astype(np.float16)
    idx, w = hi.moe_router(cuda(xn), cuda(Wr), k, 1)
    assert host(idx).tolist() == [[2, 5]] * 4
    check("moe router tie weights", host(w), np.full((4, 2), 0.5), 1e-6)


def test_moe_grouped_path_graph_replay(hi, O):
    """The grouped path launches the sort, two grouped GEMMs (the first gathering its rows through
    the tile DMA) and the combine with no host round trip, so it can be captured; every replay is
    checked, with eager work between."""
    import torch
    r = rng(420)
    E, k, H, I, flags = 32, 8, 1024, 512, 3
    M = 64
    Wr, wgu, wdn = rn(r, E, H, s=0.05), rn(r, E, 2 * I, H, s=0.02), rn(r, E, H, I, s=0.02)
    xn, x0 = rn(r, M, H), rn(r, M, H)
    xn_d, wgu_d, wdn_d = cuda(xn), cuda(wgu), cuda(wdn)
    idx_d, w_d = hi.moe_router(xn_d, cuda(Wr), k, flags)
    ref = O.moe_experts(xn, wgu, wdn, host(idx_d), host(w_d), x0.copy(), flags, 0.22)
    x = cuda(x0)
    work = torch.empty(hi.lib.hi_moe_work_bytes(M, k, E, H, I), dtype=torch.uint8, device="cuda")

    def run():
        hi.check_rc(hi.lib.hi_moe_experts(hi.ptr(xn_d), H, hi.ptr(wgu_d), hi.ptr(wdn_d), hi.ptr(idx_d), hi.ptr(w_d), M, E, k, H, I,
                                     flags, 0.22, hi.ptr(x), H, 2, hi.ptr(work), hi.cur_stream()), "moe_experts")
    run()
    torch.cuda.synchronize()
    check("grouped eager", host(x), ref, 4e-3, 4e-3)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    for _ in range(3):
        x.copy_(cuda(x0))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        check("grouped graph replay", host(x), ref, 4e-3, 4e-3)
        hi.moe_experts(xn_d, wgu_d, wdn_d, idx_d, w_d, cuda(x0), flags, 0.22, 2)  # eager work between replays


def test_moe_out_of_range_expert_ids_contribute_nothing(hi, O):
    r = rng(430)
    E, k, H, I, flags = 8, 2, 512, 256, 1
    M = 12
    wgu, wdn = rn(r, E, 2 * I, H, s=0.02), rn(r, E, H, I, s=0.02)
    xn, x0 = rn(r, M, H), rn(r, M, H)
    idx = r.integers(0, E, (M, k)).astype(np.int32)
    w = r.random((M, k)).astype(np.float32)
    idx[1, 0], idx[5, 1], idx[7, 0] = -1, E, 1000
    bad = (idx < 0) | (idx >= E)
    ref = O.moe_experts(xn, wgu, wdn, np.where(bad, 0, idx).astype(np.int32), np.where(bad, 0, w).astype(np.float32),
                        x0.copy(), flags, 1.0)
    for path in (1, 2):
        out = host(hi.moe_experts(cuda(xn), cuda(wgu), cuda(wdn), cuda(idx), cuda(w), cuda(x0), flags, 1.0, path))
        check(f"out-of-range ids path={path}", out, ref, 4e-3, 4e-3)


def test_moe_rejects_bad_arguments(hi):
    import torch
    xn = torch.zeros(2, 48, dtype=torch.float16, device="cuda")
    Wr = torch.zeros(4, 48, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        hi.moe_router(xn, Wr, 5, 1)  # k > E
    wgu = torch.zeros(4, 64, 48, dtype=torch.float16, device="cuda")
    wdn = torch.zeros(4, 48, 32, dtype=torch.float16, device="cuda")
    idx = torch.zeros(2, 1, dtype=torch.int32, device="cuda")
    w = torch.ones(2, 1, dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError):
        hi.moe_experts(xn, wgu, wdn, idx, w, xn.clone(), 1)  # H = 48 is not a multiple of 32


@pytest.mark.parametrize("name,E,k,H,I,flags,scale", LAYERS, ids=[l[0] for l in LAYERS])
def test_moe_route_experts_is_router_then_experts(hi, name, E, k, H, I, flags, scale):
    """hi_moe_route_experts (router inside the gate/up launch up to HIPINFER_GEMV_MAX rows, the two
    calls above it) gives the same bits as hi_moe_router followed by hi_moe_experts(path 0): the
    routing (indices, order, weights) and the updated residual, at M on both sides of the limit."""
    r = rng(440 + E)
    Wr = cuda(rn(r, E, H, s=0.05))
    wgu, wdn = cuda(rn(r, E, 2 * I, H, s=0.02)), cuda(rn(r, E, H, I, s=0.02))
    for M in [1, 2, 3, 4, 5, 37, 300]:
        xn, x0 = cuda(rn(r, M, H)), cuda(rn(r, M, H))
        idx2, w2 = hi.moe_router(xn, Wr, k, flags)
        ref = host(hi.moe_experts(xn, wgu, wdn, idx2, w2, x0.clone(), flags, scale, 0))
        x = x0.clone()
        idx, w = hi.moe_route_experts(xn, Wr, wgu, wdn, k, x, flags, scale)
        assert np.array_equal(host(idx), host(idx2)), f"{name} M={M}: routing differs"
        assert np.array_equal(host(w).view(np.uint32), host(w2).view(np.uint32)), f"{name} M={M}: weights differ"
        assert np.array_equal(host(x).view(np.uint16), ref.view(np.uint16)), f"{name} M={M}: output differs"


def test_moe_route_experts_graph_replay(hi):
    """The fused decode call captured in a graph: every replay, with eager work between, equals the
    eager two-call result bit for bit."""
    import torch
    r = rng(450)
    E, k, H, I, flags, M = 32, 8, 1024, 512, 3, 1
    Wr, wgu, wdn = cuda(rn(r, E, H, s=0.05)), cuda(rn(r, E, 2 * I, H, s=0.02)), cuda(rn(r, E, H, I, s=0.02))
    xn, x0 = cuda(rn(r, M, H)), cuda(rn(r, M, H))
    idx2, w2 = hi.moe_router(xn, Wr, k, flags)
    ref = host(hi.moe_experts(xn, wgu, wdn, idx2, w2, x0.clone(), flags, 0.22, 0))
    x = x0.clone()
    idx = torch.empty(M, k, dtype=torch.int32, device="cuda")
    w = torch.empty(M, k, dtype=torch.float32, device="cuda")
    work = torch.zeros(hi.lib.hi_moe_work_bytes(M, k, E, H, I), dtype=torch.uint8, device="cuda")

    def run():
        hi.check_rc(hi.lib.hi_moe_route_experts(hi.ptr(xn), H, hi.ptr(Wr), hi.ptr(wgu), hi.ptr(wdn), M, E, k, H, I, flags, 0.22,
                                           hi.ptr(x), H, hi.ptr(idx), hi.ptr(w), hi.ptr(work), hi.cur_stream()), "moe_route_experts")
    run()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    for _ in range(3):
        x.copy_(x0)
        idx.fill_(-7)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(x).view(np.uint16), ref.view(np.uint16))
        assert np.array_equal(host(idx), host(idx2))
        hi.moe_route_experts(xn, Wr, wgu, wdn, k, x0.clone(), flags, 0.22)  # eager work between replays


def test_moe_route_experts_grouped_graph_replay(hi):
    """Above the GEMV row limit (router, sort, two grouped GEMMs with gathered A rows and scattered
    C rows, combine): captured in a graph and replayed, with eager calls on the same work buffer
    between replays, every result equals the router + grouped experts bit for bit."""
    import torch
    r = rng(455)
    E, k, H, I, flags, M = 32, 8, 1024, 512, 3, 256
    Wr, wgu, wdn = cuda(rn(r, E, H, s=0.05)), cuda(rn(r, E, 2 * I, H, s=0.02)), cuda(rn(r, E, H, I, s=0.02))
    xn, x0 = cuda(rn(r, M, H)), cuda(rn(r, M, H))
    idx2, w2 = hi.moe_router(xn, Wr, k, flags)
    ref = host(hi.moe_experts(xn, wgu, wdn, idx2, w2, x0.clone(), flags, 0.22, 2))
    x = x0.clone()
    idx = torch.empty(M, k, dtype=torch.int32, device="cuda")
    w = torch.empty(M, k, dtype=torch.float32, device="cuda")
    work = torch.zeros(hi.lib.hi_moe_work_bytes(M, k, E, H, I), dtype=torch.uint8, device="cuda")

    def run(xx):
        hi.check_rc(hi.lib.hi_moe_route_experts(hi.ptr(xn), H, hi.ptr(Wr), hi.ptr(wgu), hi.ptr(wdn), M, E, k, H, I, flags,
                                                0.22, hi.ptr(xx), H, hi.ptr(idx), hi.ptr(w), hi.ptr(work),
                                                hi.cur_stream()), "moe_route_experts")
    run(x)
    torch.cuda.synchronize()
    assert np.array_equal(host(x).view(np.uint16), ref.view(np.uint16))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run(x)
    for _ in range(3):
        x.copy_(x0)
        idx.fill_(-7)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(x).view(np.uint16), ref.view(np.uint16))
        assert np.array_equal(host(idx), host(idx2))
        xe = x0.clone()
        run(xe)  # eager work on the same buffer between replays
        torch.cuda.synchronize()
        assert np.array_equal(host(xe).view(np.uint16), ref.view(np.uint16))


def test_moe_route_experts_shared_work_across_shapes(hi):
    """One zeroed work buffer serves single-row calls of every layer shape in turn, twice round:
    the one-launch path's arrival counters live in it and carry each launch's totals to the next
    (grids of 32 to 256 blocks), and every call still equals the two calls bit for bit."""
    import torch
    r = rng(460)
    layers = []
    for name, E, k, H, I, flags, scale in LAYERS:
        layers.append((name, E, k, H, I, flags, scale, cuda(rn(r, E, H, s=0.05)), cuda(rn(r, E, 2 * I, H, s=0.02)),
                       cuda(rn(r, E, H, I, s=0.02))))
    nbytes = max(hi.lib.hi_moe_work_bytes(1, k, E, H, I) for _, E, k, H, I, *_ in layers)
    work = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    for rnd in range(2):
        for name, E, k, H, I, flags, scale, Wr, wgu, wdn in layers:
            xn, x0 = cuda(rn(r, 1, H)), cuda(rn(r, 1, H))
            idx2, w2 = hi.moe_router(xn, Wr, k, flags)
            ref = host(hi.moe_experts(xn, wgu, wdn, idx2, w2, x0.clone(), flags, scale, 0))
            x = x0.clone()
            idx = torch.empty(1, k, dtype=torch.int32, device="cuda")
            w = torch.empty(1, k, dtype=torch.float32, device="cuda")
            hi.check_rc(hi.lib.hi_moe_route_experts(hi.ptr(xn), H, hi.ptr(Wr), hi.ptr(wgu), hi.ptr(wdn), 1, E, k, H, I,
                                                    flags, scale, hi.ptr(x), H, hi.ptr(idx), hi.ptr(w), hi.ptr(work),
                                                    hi.cur_stream()), "moe_route_experts")
            assert np.array_equal(host(idx), host(idx2)), f"{name} round {rnd}: routing differs"
            assert np.array_equal(host(x).view(np.uint16), ref.view(np.uint16)), f"{name} round {rnd}: output differs"


def test_moe_route_experts_rejects_bad_arguments(hi):
    import torch
    xn = torch.zeros(1, 64, dtype=torch.float16, device="cuda")
    Wr = torch.zeros(4, 64, dtype=torch.float16, device="cuda")
    wgu = torch.zeros(4, 64, 64, dtype=torch.float16, device="cuda")
    wdn = torch.zeros(4, 64, 32, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        hi.moe_route_experts(xn, Wr, wgu, wdn, 5, xn.clone(), 1)  # k > E
    with pytest.raises(ValueError):
        hi.moe_route_experts(xn[:, :48], Wr[:, :48], wgu[:, :, :48], wdn[:, :48], 2, xn[:, :48].clone(), 1)  # H = 48


def test_moe_one_launch_timeout_is_reported(hi):
    """The one-launch path's bounded handoff wait, made to run out from the host: a zeroed work
    buffer whose expected-total words (the 8 words after the 8 arrival counters, 256 bytes apart)
    are preset far above the counters, so no block ever sees its target. Every block gives up after
    its bounded polls and exits (the call and a device synchronize succeed); the next call reports
    that output as wrong (-2) and launches nothing; later calls take the two launches and equal the
    router + experts bit for bit. Last in this file: a reported timeout turns the one-launch path
    off for the rest of the process."""
    import torch
    r = rng(470)
    E, k, H, I, flags, scale = 32, 8, 1024, 512, 3, 0.22
    Wr, wgu, wdn = cuda(rn(r, E, H, s=0.05)), cuda(rn(r, E, 2 * I, H, s=0.02)), cuda(rn(r, E, H, I, s=0.02))
    xn, x0 = cuda(rn(r, 1, H)), cuda(rn(r, 1, H))
    idx = torch.empty(1, k, dtype=torch.int32, device="cuda")
    w = torch.empty(1, k, dtype=torch.float32, device="cuda")
    work = torch.zeros(hi.lib.hi_moe_work_bytes(1, k, E, H, I), dtype=torch.uint8, device="cuda")

    def call(x):
        return hi.lib.hi_moe_route_experts(hi.ptr(xn), H, hi.ptr(Wr), hi.ptr(wgu), hi.ptr(wdn), 1, E, k, H, I, flags,
                                           scale, hi.ptr(x), H, hi.ptr(idx), hi.ptr(w), hi.ptr(work), hi.cur_stream())

    assert call(x0.clone()) == 0  # the fail word is allocated on this first, ordinary call
    torch.cuda.synchronize()
    work.zero_()
    work.view(torch.int32)[8 * 64:8 * 64 + 8] = 1 << 20  # expected totals far above the zero counters
    print("moe one-launch: forcing the bounded handoff wait to run out", flush=True)
    assert call(x0.clone()) == 0
    torch.cuda.synchronize()  # every block gave up and exited
    assert call(x0.clone()) == -2, "the timed-out call was not reported"
    work.zero_()
    idx2, w2 = hi.moe_router(xn, Wr, k, flags)
    ref = host(hi.moe_experts(xn, wgu, wdn, idx2, w2, x0.clone(), flags, scale, 0))
    for _ in range(2):
        x = x0.clone()
        assert call(x) == 0
        assert np.array_equal(host(idx), host(idx2))
        assert np.array_equal(host(x).view(np.uint16), ref.view(np.uint16))
