"""GPU parity of the engine's prefill and of the batched (GEMM-path) decode step
(hipinfer_amd.engine.DecodeStep; the reference's prefill / prefill_layers, src/api.cu:1668-1845,
and decode_step's GEMM branch, api.cu:1914-1940), on a small random model, against the same
computation chained from the CPU oracle.

Prefill: a prompt in two chunks (max_prefill smaller than the prompt), then a continuation at
p0 > 0 into the same slot, in a second slot too; every layer's K/V cache rows, the last position's
logits and the greedy token are checked, then decode steps continue from the prefilled caches on
the GEMV path. Batched decode: 12 sequences (above the GEMV limit) through the GEMM path, eager
and as graph replays.
"""
import numpy as np
import pytest

from tests._util import check, cuda, gpu, host, rng
from tests.test_decode_step import CFG, host_w, make_weights, oracle_step, to_device

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


def _wsplit(Wd, k):
    v = host_w(Wd, k)
    return (v[0], v[1]) if isinstance(v, tuple) else (v, None)


def oracle_prefill(O, c, Wd, tokens, p0, slot, kc, vc, cs):
    """The prefill chain on the oracle; kc / vc (lists over layers of [slots, Hkv, S, D]) in place."""
    Hq, Hkv, D, eps = c["Hq"], c["Hkv"], c["D"], c["eps"]
    T = len(tokens)
    x = host(Wd["embed"])[np.asarray(tokens)].copy()
    for l, ly in enumerate(Wd["layers"]):
        xn = O.rmsnorm(x, host(ly["n1"]), eps)
        Wq, sq = _wsplit(ly, "qkv")
        qkv = O.gemm(xn, Wq, bias=host(ly["bqkv"]), scales=sq)
        O.rope_cache(qkv, Hq, Hkv, cs, kc[l], vc[l], pos_base=p0, slot_base=slot)
        att = O.flash_prefill(np.ascontiguousarray(qkv[:, :Hq * D]), kc[l][slot], vc[l][slot], T, p0, Hq, Hkv)
        Wo, so = _wsplit(ly, "o")
        x = O.gemm(att, Wo, out=x, epi=1, scales=so)
        xn = O.rmsnorm(x, host(ly["n2"]), eps)
        Wg, sg = _wsplit(ly, "gate_up")
        act = O.gemm(xn, Wg, epi=2, scales=sg)
        Wdn, sdn = _wsplit(ly, "down")
        x = O.gemm(act, Wdn, out=x, epi=1, scales=sdn)
    Wl, sl = _wsplit(Wd, "lm")
    logits = O.gemv(x[-1:], Wl, normw=host(Wd["nf"]), eps=eps, scales=sl)
    return logits, int(O.argmax(logits)[0])


def oracle_step_gemm(O, c, Wd, tok, pos, kc, vc, cs):
    """The GEMM-path decode step on the oracle (row b = slot b)."""
    Hq, Hkv, D, eps = c["Hq"], c["Hkv"], c["D"], c["eps"]
    x = host(Wd["embed"])[tok].copy()
    for l, ly in enumerate(Wd["layers"]):
        xn = O.rmsnorm(x, host(ly["n1"]), eps)
        Wq, sq = _wsplit(ly, "qkv")
        qkv = O.gemm(xn, Wq, bias=host(ly["bqkv"]), scales=sq)
        O.rope_cache(qkv, Hq, Hkv, cs, kc[l], vc[l], pos=pos)
        att = O.decode_attn(np.ascontiguousarray(qkv[:, :Hq * D]), kc[l], vc[l], pos, Hq, Hkv)
        Wo, so = _wsplit(ly, "o")
        x = O.gemm(att, Wo, out=x, epi=1, scales=so)
        xn = O.rmsnorm(x, host(ly["n2"]), eps)
        Wg, sg = _wsplit(ly, "gate_up")
        act = O.gemm(xn, Wg, epi=2, scales=sg)
        Wdn, sdn = _wsplit(ly, "down")
        x = O.gemm(act, Wdn, out=x, epi=1, scales=sdn)
    Wl, sl = _wsplit(Wd, "lm")
    logits = O.gemm(O.rmsnorm(x, host(Wd["nf"]), eps), Wl, scales=sl)
    return logits, O.argmax(logits)


def clear_top(logits, tol=4e-2):
    lg = logits.astype(np.float64)
    top2 = np.sort(lg, axis=-1)[..., -2:]
    return (top2[..., 1] - top2[..., 0]) > tol


@pytest.mark.parametrize("q8", [False, True], ids=["fp16", "int8"])
def test_prefill_then_decode_vs_oracle_chain(hi, O, q8):
    import torch
    from hipinfer_amd.engine import DecodeStep
    c = CFG
    r = rng(1300 + q8)
    Wd = to_device(hi, make_weights(r, c), q8)
    B, S = 2, 160
    ds = DecodeStep(c, Wd, B, S, max_prefill=24)
    cs = host(ds.cs)
    kc = [np.zeros((B, c["Hkv"], S, c["D"]), np.float16) for _ in range(c["L"])]
    vc = [np.zeros_like(k) for k in kc]
    prompts = [(1, r.integers(0, c["V"], 37).tolist(), 0),   # two chunks
               (1, r.integers(0, c["V"], 20).tolist(), 37),  # continuation of slot 1
               (0, r.integers(0, c["V"], 5).tolist(), 0)]    # a short prompt in slot 0
    for slot, toks, p0 in prompts:
        got_tok = ds.prefill(slot, toks, p0)
        torch.cuda.synchronize()
        ref_logits, ref_tok = oracle_prefill(O, c, Wd, toks, p0, slot, kc, vc, cs)
        tag = f"{'int8' if q8 else 'fp16'} slot {slot} p0 {p0} T {len(toks)}"
        check(f"{tag} last-position logits", host(ds.logits[slot:slot + 1]), ref_logits, 2e-2, 2e-2)
        if clear_top(ref_logits)[0]:
            assert got_tok == ref_tok, (tag, got_tok, ref_tok)
        assert int(host(ds.pos)[slot]) == p0 + len(toks)
        for l in range(c["L"]):
            end = p0 + len(toks)
            check(f"{tag} layer {l} K rows", host(ds.kc[l][slot, :, p0:end]), kc[l][slot, :, p0:end], 2e-2, 2e-2)
            check(f"{tag} layer {l} V rows", host(ds.vc[l][slot, :, p0:end]), vc[l][slot, :, p0:end], 2e-2, 2e-2)
        # both continue from the oracle's caches and token
        for l in range(c["L"]):
            ds.kc[l].copy_(torch.from_numpy(kc[l]))
            ds.vc[l].copy_(torch.from_numpy(vc[l]))
        ds.tok[slot:slot + 1].fill_(ref_tok)
    # decode (GEMV path) from the prefilled caches: slot 1 at position 57, slot 0 at 5
    tok = host(ds.tok).astype(np.int32)
    pos = host(ds.pos).astype(np.int32)
    assert list(pos) == [5, 57]
    for step in range(3):
        ref_logits, ref_tok = oracle_step(O, c, Wd, tok, pos, kc, vc, cs)
        ds.step()
        torch.cuda.synchronize()
        check(f"decode after prefill step {step}", host(ds.logits), ref_logits, 2e-2, 2e-2)
        clear = clear_top(ref_logits)
        assert np.array_equal(host(ds.tok)[clear], ref_tok[clear])
        tok, pos = ref_tok, pos + 1
        ds.tok.copy_(torch.from_numpy(tok))
        for l in range(c["L"]):
            ds.kc[l].copy_(torch.from_numpy(kc[l]))
            ds.vc[l].copy_(torch.from_numpy(vc[l]))


@pytest.mark.parametrize("q8", [False, True], ids=["fp16", "int8"])
def test_batched_decode_gemm_path_vs_oracle_chain(hi, O, q8):
    """12 sequences: the GEMM path (RMSNorm, GEMM + bias, RoPE/cache, decode attention, GEMMs); the
    first step eager (tunes the tiles), then graph replays."""
    import torch
    from hipinfer_amd.engine import DecodeStep
    c = CFG
    r = rng(1400 + q8)
    Wd = to_device(hi, make_weights(r, c), q8)
    B, S = 12, 96
    ds = DecodeStep(c, Wd, B, S)
    assert ds.gemm_path
    cs = host(ds.cs)
    p0 = r.integers(1, 60, B).astype(np.int32)
    kc = [r.standard_normal((B, c["Hkv"], S, c["D"])).astype(np.float16) for _ in range(c["L"])]
    vc = [r.standard_normal((B, c["Hkv"], S, c["D"])).astype(np.float16) for _ in range(c["L"])]
    for l in range(c["L"]):
        for b in range(B):
            kc[l][b, :, p0[b]:] = 0
            vc[l][b, :, p0[b]:] = 0
        ds.kc[l].copy_(torch.from_numpy(kc[l]))
        ds.vc[l].copy_(torch.from_numpy(vc[l]))
    tok = r.integers(0, c["V"], B).astype(np.int32)
    pos = p0.copy()
    ds.tok.copy_(torch.from_numpy(tok))
    ds.pos.copy_(torch.from_numpy(pos))
    graph = None
    for step in range(4):
        ref_logits, ref_tok = oracle_step_gemm(O, c, Wd, tok, pos, kc, vc, cs)
        if step == 0:
            ds.step()
        else:
            if graph is None:
                graph = ds.capture()
            graph.replay()
        torch.cuda.synchronize()
        tag = f"{'int8' if q8 else 'fp16'} B={B} step {step}"
        check(f"{tag} logits", host(ds.logits), ref_logits, 2e-2, 2e-2)
        for l in range(c["L"]):
            got_k = np.stack([host(ds.kc[l][b, :, pos[b]]) for b in range(B)])
            check(f"{tag} layer {l} new K rows", got_k, np.stack([kc[l][b, :, pos[b]] for b in range(B)]), 2e-2, 2e-2)
        clear = clear_top(ref_logits)
        assert np.array_equal(host(ds.tok)[clear], ref_tok[clear]), tag
        assert np.array_equal(host(ds.pos), pos + 1)
        tok, pos = ref_tok, pos + 1
        ds.tok.copy_(torch.from_numpy(tok))
        for l in range(c["L"]):
            ds.kc[l].copy_(torch.from_numpy(kc[l]))
            ds.vc[l].copy_(torch.from_numpy(vc[l]))
