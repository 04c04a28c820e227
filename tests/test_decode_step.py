"""GPU parity of a whole greedy decode step (hipinfer_amd.engine.DecodeStep: embed, per layer
QKV+bias+RoPE+KV write, decode attention, o_proj + residual, RMSNorm + gate/up + SwiGLU, down +
residual, final RMSNorm + lm_head, argmax; the reference's decode_step, src/api.cu:1891-1952), on
a small random model with pre-filled caches, against the same step chained from the CPU oracle.

The first step runs eagerly, the following ones as replays of one captured hipGraph, so the
device-side token / position bookkeeping is covered too. Each step's logits must match within
tolerance, the new K/V cache rows too; the greedy tokens must match wherever the oracle's top two
logits are apart by more than the tolerance (elsewhere both paths continue from the oracle's).
"""
import numpy as np
import pytest

from tests._util import check, cuda, gpu, host, rng

pytestmark = gpu

CFG = dict(H=512, Hq=8, Hkv=2, D=64, I=1024, V=2048, L=2, eps=1e-5, theta=10000.0)


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


def make_weights(r, c):
    H, Hq, Hkv, D, I, V = (c[k] for k in ("H", "Hq", "Hkv", "D", "I", "V"))
    w = lambda n, k, sd=0.05: (r.standard_normal((n, k)) * sd).astype(np.float16)
    nrm = lambda: (r.random(H) + 0.5).astype(np.float16)
    layers = []
    for _ in range(c["L"]):
        layers.append({"qkv": w((Hq + 2 * Hkv) * D, H), "bqkv": (r.standard_normal((Hq + 2 * Hkv) * D) * 0.1).astype(np.float16),
                       "o": w(H, Hq * D), "gate_up": w(2 * I, H), "down": w(H, I, 0.03), "n1": nrm(), "n2": nrm()})
    return {"embed": (r.standard_normal((V, H))).astype(np.float16), "lm": w(V, H), "nf": nrm(), "layers": layers}


def to_device(hi, W, q8):
    def mat(a):
        if not q8:
            return cuda(a)
        return hi.quantize_rows(cuda(a))
    return {"embed": cuda(W["embed"]), "lm": mat(W["lm"]), "nf": cuda(W["nf"]),
            "layers": [{k: (mat(v) if k in ("qkv", "o", "gate_up", "down") else cuda(v)) for k, v in ly.items()}
                       for ly in W["layers"]]}


def host_w(Wd, k):
    """The host copy of a device weight: fp16, or (int8, scales) for the oracle's int8 path."""
    v = Wd[k]
    return (host(v[0]), host(v[1])) if isinstance(v, tuple) else host(v)


def oracle_step(O, c, Wd, tok, pos, kc, vc, cs):
    H, Hq, Hkv, D = c["H"], c["Hq"], c["Hkv"], c["D"]
    B = tok.shape[0]
    x = host(Wd["embed"])[tok].copy()
    for l, ly in enumerate(Wd["layers"]):
        Wq = host_w(ly, "qkv")
        q = np.zeros((B, Hq * D), np.float16)
        O.gemv_qkv_rope(x, Wq[0] if isinstance(Wq, tuple) else Wq, host(ly["n1"]), Hq, Hkv, cs, pos, kc[l], vc[l], q,
                        bias=host(ly["bqkv"]), eps=c["eps"], scales=Wq[1] if isinstance(Wq, tuple) else None)
        att = O.decode_attn(q, kc[l], vc[l], pos, Hq, Hkv)
        for name, src, epi, nw in [("o", att, 1, None), ("gate_up", None, 2, ly["n2"]), ("down", None, 1, None)]:
            Wm = host_w(ly, name)
            Wm, s = (Wm[0], Wm[1]) if isinstance(Wm, tuple) else (Wm, None)
            if name == "o":
                x = O.gemv(att, Wm, out=x, epi=1, scales=s)
            elif name == "gate_up":
                act = O.gemv(x, Wm, epi=2, normw=host(nw), eps=c["eps"], scales=s)
            else:
                x = O.gemv(act, Wm, out=x, epi=1, scales=s)
    Wl = host_w(Wd, "lm")
    Wl, s = (Wl[0], Wl[1]) if isinstance(Wl, tuple) else (Wl, None)
    logits = O.gemv(x, Wl, normw=host(Wd["nf"]), eps=c["eps"], scales=s)
    return logits, O.argmax(logits)


@pytest.mark.parametrize("mask", [None, 7, 2], ids=["rule_paths", "gemm_gu_down_lm", "gemm_down"])
@pytest.mark.parametrize("q8", [False, True], ids=["fp16", "int8"])
def test_decode_step_vs_oracle_chain(hi, O, q8, mask):
    """mask: the projections a 2-sequence step runs on the GEMM path (engine.GU_GEMM | DOWN_GEMM |
    LM_GEMM), or None for the engine's shape rule; every choice must match the oracle."""
    import torch
    from hipinfer_amd.engine import DecodeStep
    r = rng(800 + q8)
    c = CFG
    B, S = 2, 64
    Wd = to_device(hi, make_weights(r, c), q8)
    ds = DecodeStep(c, Wd, B, S, small_gemm=mask)
    p0 = np.array([5, 17], np.int32)
    kc = [r.standard_normal((B, c["Hkv"], S, c["D"])).astype(np.float16) for _ in range(c["L"])]
    vc = [r.standard_normal((B, c["Hkv"], S, c["D"])).astype(np.float16) for _ in range(c["L"])]
    for l in range(c["L"]):  # the "prompt": random keys / values before p0
        for b in range(B):
            kc[l][b, :, p0[b]:] = 0
            vc[l][b, :, p0[b]:] = 0
        ds.kc[l].copy_(torch.from_numpy(kc[l]))
        ds.vc[l].copy_(torch.from_numpy(vc[l]))
    tok = np.array([3, 1999], np.int32)
    pos = p0.copy()
    ds.tok.copy_(torch.from_numpy(tok))
    ds.pos.copy_(torch.from_numpy(pos))
    cs = host(ds.cs)
    graph = None
    for step in range(5):
        ref_logits, ref_tok = oracle_step(O, c, Wd, tok, pos, kc, vc, cs)
        if step == 0:
            ds.step()
        else:
            if graph is None:
                graph = ds.capture()
            graph.replay()
        torch.cuda.synchronize()
        check(f"{'int8' if q8 else 'fp16'} step {step} logits", host(ds.logits), ref_logits, 2e-2, 2e-2)
        for l in range(c["L"]):
            for b in range(B):
                check(f"step {step} layer {l} new K/V row b={b}", host(ds.kc[l][b, :, pos[b]]), kc[l][b, :, pos[b]],
                      1e-2, 1e-2)
                check(f"step {step} layer {l} new V row b={b}", host(ds.vc[l][b, :, pos[b]]), vc[l][b, :, pos[b]],
                      1e-2, 1e-2)
        got_tok = host(ds.tok)
        lg = ref_logits.astype(np.float64)
        top2 = np.sort(lg, axis=1)[:, -2:]
        clear = (top2[:, 1] - top2[:, 0]) > 4e-2
        assert np.array_equal(got_tok[clear], ref_tok[clear]), (step, got_tok, ref_tok)
        assert np.array_equal(host(ds.pos), pos + 1), (step, host(ds.pos), pos)
        # both continue from the oracle's token and caches
        tok, pos = ref_tok, pos + 1
        ds.tok.copy_(torch.from_numpy(tok))
        for l in range(c["L"]):
            ds.kc[l].copy_(torch.from_numpy(kc[l]))
            ds.vc[l].copy_(torch.from_numpy(vc[l]))
