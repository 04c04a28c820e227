"""Benchmark of the matmul hot path on one MI355X (BASELINE.json metric, config C2).

A step is one decode token of Llama-3.1-8B at batch 1 through every matmul of the model: per
layer the fused RMSNorm + QKV + RoPE + KV-write GEMV, o_proj + residual, fused RMSNorm + gate/up +
SwiGLU, down + residual (the reference's decode_step order, api.cu:1891-1952, attention aside),
then the RMSNorm + lm_head GEMV. All 32 layers' distinct weight sets (15.0 GB fp16, 7.5 GB int8 +
row scales) are streamed once per token from HBM, so the 256 MB MALL cannot serve them. The token
is captured once as a hipGraph and replayed. Weights ~N(0, 0.02), activations and norm weights
seeded; everything is generated on the GPU (synthetic data, random-init weights of the
architecture).

value: fp16 decode-GEMV throughput in GB/s = algorithmic weight bytes per token / time per token.
Also reported: the int8 token, each GEMV kind alone, the prefill GEMM (C3) when built, the
dominant kernel's roofline (gate/up GEMV, timed with HIP events on the stream it runs on), and the
CPU baseline (the oracle's GEMV restatement on one layer, timed on the host cores).

python bench.py [--gpus 1] [--steps 20] [--warmup 3]
"""
import argparse
import json
import os
import statistics
import sys
import time

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, datasheet
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, datasheet

# Llama-3.1-8B
H, HQ, HKV, D, I, V, L = 4096, 32, 8, 128, 14336, 128256, 32
QKV = (HQ + 2 * HKV) * D
SHAPES = {"qkv": (QKV, H), "o": (H, HQ * D), "gate_up": (2 * I, H), "down": (H, I)}
SEED = 1219 + 1


def weight_bytes(q8):
    """Algorithmic bytes per token the reference counts (bench.py:147,234): N*K*w + 2N scales."""
    w = 1 if q8 else 2
    per_layer = sum(N * K * w + (2 * N if q8 else 0) for N, K in SHAPES.values())
    return per_layer * L + V * H * w + (2 * V if q8 else 0)


def act_bytes():
    """Activation/output bytes per token on top of the weights (x reads, out writes, residual reads,
    the K/V cache writes), each counted once per GEMV."""
    per_layer = (H * 2 + QKV * 2) + (HQ * D * 2 + 2 * H * 2) + (H * 2 + I * 2) + (I * 2 + 2 * H * 2)
    return per_layer * L + H * 2 + V * 2


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Model:
    def __init__(self, torch, hi, q8_too=True):
        self.torch, self.hi = torch, hi
        dev = "cuda"
        g = torch.Generator(device=dev)
        g.manual_seed(SEED)

        def w(N, K):
            return torch.empty(N, K, dtype=torch.float16, device=dev).normal_(0.0, 0.02, generator=g)

        def nrm(n):
            return (torch.rand(n, generator=g, device=dev) + 0.5).half()

        self.layers = []
        for _ in range(L):
            ly = {k: w(*s) for k, s in SHAPES.items()}
            ly["n1"], ly["n2"] = nrm(H), nrm(H)
            self.layers.append(ly)
        self.lm = w(V, H)
        self.nf = nrm(H)
        self.q8 = None
        if q8_too:
            self.q8 = []
            for ly in self.layers:
                self.q8.append({k: hi.quantize_rows(ly[k]) for k in SHAPES})
            self.lm_q = hi.quantize_rows(self.lm)
        self.max_seq = 64
        self.kc = [torch.zeros(1, HKV, self.max_seq, D, dtype=torch.float16, device=dev) for _ in range(L)]
        self.vc = [torch.zeros_like(k) for k in self.kc]
        ang = torch.arange(self.max_seq, device=dev).float()[:, None] * (
            1.0 / 500000.0 ** (torch.arange(0, D, 2, device=dev).float() / D))[None, :]
        self.cs = torch.stack([ang.cos(), ang.sin()], -1).half().contiguous()
        self.pos = torch.tensor([7], dtype=torch.int32, device=dev)
        self.x = torch.randn(1, H, generator=g, device=dev).half()
        self.x0 = self.x.clone()
        self.q = torch.empty(1, HQ * D, dtype=torch.float16, device=dev)
        self.act = torch.empty(1, I, dtype=torch.float16, device=dev)
        self.logits = torch.empty(1, V, dtype=torch.float16, device=dev)
        torch.cuda.synchronize()

    def _w(self, l, name, q8):
        if not q8:
            return self.layers[l][name], None
        return self.q8[l][name]

    def token(self, q8):
        """One decode token through every matmul of the model (fused epilogues as the engine runs them)."""
        hi = self.hi
        self.x.copy_(self.x0)
        for l in range(L):
            W, s = self._w(l, "qkv", q8)
            hi.gemv_qkv_rope(self.x, W, self.layers[l]["n1"], HQ, HKV, self.cs, self.pos, self.kc[l], self.vc[l], self.q,
                             scales=s)
            W, s = self._w(l, "o", q8)
            hi.gemv(self.q, W, out=self.x, epi=1, scales=s)
            W, s = self._w(l, "gate_up", q8)
            hi.gemv(self.x, W, out=self.act, normw=self.layers[l]["n2"], epi=2, scales=s)
            W, s = self._w(l, "down", q8)
            hi.gemv(self.act, W, out=self.x, epi=1, scales=s)
        W, s = (self.lm, None) if not q8 else self.lm_q
        hi.gemv(self.x, W, out=self.logits, normw=self.nf, scales=s)

    def one_kind(self, kind, q8):
        """The 32 layers' GEMVs of one kind back to back (or the lm_head 4 times)."""
        hi = self.hi
        if kind == "lm_head":
            W, s = (self.lm, None) if not q8 else self.lm_q
            for _ in range(4):
                hi.gemv(self.x, W, out=self.logits, normw=self.nf, scales=s)
            return 4
        for l in range(L):
            W, s = self._w(l, kind, q8)
            if kind == "qkv":
                hi.gemv_qkv_rope(self.x, W, self.layers[l]["n1"], HQ, HKV, self.cs, self.pos, self.kc[l], self.vc[l],
                                 self.q, scales=s)
            elif kind == "o":
                hi.gemv(self.q, W, out=self.x, epi=1, scales=s)
            elif kind == "gate_up":
                hi.gemv(self.x, W, out=self.act, normw=self.layers[l]["n2"], epi=2, scales=s)
            else:
                hi.gemv(self.act, W, out=self.x, epi=1, scales=s)
        return L


# Llama-3.2-3B prefill
P_H, P_HQ, P_HKV, P_D, P_I, P_L = 3072, 24, 8, 128, 8192, 28
P_SHAPES = {"qkv": ((P_HQ + 2 * P_HKV) * P_D, P_H), "o": (P_H, P_HQ * P_D), "gate_up": (2 * P_I, P_H),
            "down": (P_H, P_I)}


class PrefillModel:
    """All 28 layers' projection weights of Llama-3.2-3B (5.6 GB fp16, plus int8 copies), so a
    step through every layer streams distinct weights like a real prefill chunk."""

    def __init__(self, torch, hi, q8_too=True):
        self.torch, self.hi = torch, hi
        g = torch.Generator(device="cuda")
        g.manual_seed(SEED + 1)
        self.layers = [{k: torch.empty(*s, dtype=torch.float16, device="cuda").normal_(0.0, 0.02, generator=g)
                        for k, s in P_SHAPES.items()} for _ in range(P_L)]
        self.q8 = [{k: hi.quantize_rows(ly[k]) for k in P_SHAPES} for ly in self.layers] if q8_too else None
        self.gen = g

    def buffers(self, M):
        t = self.torch
        x = t.randn(M, P_H, generator=self.gen, device="cuda").half()
        return {"x": x, "x0": x.clone(), "qkv": t.empty(M, P_SHAPES["qkv"][0], dtype=t.float16, device="cuda"),
                "act": t.empty(M, P_I, dtype=t.float16, device="cuda")}

    def layer_pass(self, b, q8, kinds=("qkv", "o", "gate_up", "down")):
        """Every layer's four GEMMs in the engine's order (attn_rows / mlp_rows, api.cu:1668-1718):
        QKV (store), o_proj + residual (the attention output is stood in by the q columns), gate/up
        + SwiGLU, down + residual."""
        hi = self.hi
        b["x"].copy_(b["x0"])
        for l in range(P_L):
            w = (lambda k: (self.layers[l][k], None)) if not q8 else (lambda k: self.q8[l][k])
            if "qkv" in kinds:
                W, s = w("qkv")
                hi.gemm(b["x"], W, out=b["qkv"], scales=s)
            if "o" in kinds:
                W, s = w("o")
                hi.gemm(b["qkv"][:, :P_HQ * P_D], W, out=b["x"], epi=1, scales=s)
            if "gate_up" in kinds:
                W, s = w("gate_up")
                hi.gemm(b["x"], W, out=b["act"], epi=2, scales=s)
            if "down" in kinds:
                W, s = w("down")
                hi.gemm(b["act"], W, out=b["x"], epi=1, scales=s)


def decode_step_bench(torch, hi, model, steps, ctxs=(1024, 4096)):
    """The whole greedy decode step of Llama-3.1-8B at batch 1 (hipinfer_amd.engine.DecodeStep:
    embed, 32 x [QKV+RoPE+KV write, decode attention, o + residual, gate/up + SwiGLU, down +
    residual], lm_head, argmax; the reference's decode_step, api.cu:1891-1952) over a KV cache
    already holding ctx positions, captured once as a hipGraph and replayed; plus the 32 layers'
    decode attention alone at each context (the kernel's HBM roofline: every cached K and V byte of
    the context is read once per layer)."""
    from hipinfer_amd.engine import DecodeStep
    g = torch.Generator(device="cuda")
    g.manual_seed(SEED + 20)
    embed = torch.empty(V, H, dtype=torch.float16, device="cuda").normal_(0.0, 1.0, generator=g)
    cfg = dict(H=H, Hq=HQ, Hkv=HKV, D=D, I=I, V=V, L=L, eps=1e-5, theta=500000.0)
    max_seq = max(ctxs) + 2 * steps + 16
    res = {"config": "Llama-3.1-8B greedy decode step, batch 1, KV cache of ctx positions (synthetic), hipGraph replay"}
    for q8 in ([False, True] if model.q8 is not None else [False]):
        W = engine_weights(model, embed, q8)
        ds = DecodeStep(cfg, W, 1, max_seq)
        for k in ds.kc + ds.vc:
            k.normal_(0.0, 1.0, generator=g)
        ds.pos.fill_(min(ctxs) - 1)
        ds.step()  # eager first step: kernel attributes and occupancy queries happen outside capture
        torch.cuda.synchronize()
        gr = ds.capture()
        for ctx in ctxs:
            ds.pos.fill_(ctx - 1)
            ds.tok.fill_(1)
            ms, _ = time_graph(torch, gr, steps, 2)
            kv = L * HKV * (ctx + 2 + steps // 2) * D * 2 * 2  # K and V bytes read per token (mean context)
            wb = weight_bytes(q8) + H * 2  # + the embedding row
            gbs = (wb + kv) / (ms * 1e-3) / 1e9
            res[f"ctx{ctx}_{'int8' if q8 else 'fp16'}"] = {
                "ms_per_token": round(ms, 4), "tokens_per_s": round(1e3 / ms, 1),
                "bytes_per_token": wb + kv, "GB/s": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1)}
        if not q8:
            # decode attention alone, the 32 layers back to back
            for ctx in ctxs:
                ds.pos.fill_(ctx - 1)

                def attn():
                    for l in range(L):
                        hi.decode_attn(ds.q, ds.kc[l], ds.vc[l], ds.pos, HQ, HKV, out=ds.att, work=ds.work)
                ga = capture(torch, attn)
                ms, _ = time_graph(torch, ga, steps, 2)
                us = ms * 1e3 / L
                b = HKV * ctx * D * 2 * 2 + HQ * D * 2 * 2
                res[f"attention_ctx{ctx}"] = {"us_per_layer": round(us, 2), "bytes_per_layer": b,
                                             "GB/s": round(b / us / 1e3, 1),
                                             "pct_hbm_peak": round(100 * b / us / 1e3 / HBM_PEAK_GBS, 1)}
                del ga
        del gr, ds
        torch.cuda.empty_cache()
    del embed
    torch.cuda.empty_cache()
    return res


def engine_weights(model, embed, q8):
    """The bench model's layer weights in the engine's layout (fp16, or (int8, scales))."""
    layers = []
    for l in range(L):
        ly = {k: (model.layers[l][k] if not q8 else model.q8[l][k]) for k in SHAPES}
        ly.update(n1=model.layers[l]["n1"], n2=model.layers[l]["n2"], bqkv=None)
        layers.append(ly)
    return {"embed": embed, "lm": model.lm if not q8 else model.lm_q, "nf": model.nf, "layers": layers}


def engine_bench(torch, hi, model, steps, T=1024, batches=(4, 8, 16, 32, 64), ctx=1024):
    """Llama-3.1-8B through the engine (hipinfer_amd.engine.DecodeStep): the prefill of a T-token
    prompt into one cache slot (embed, 32 x [RMSNorm, QKV GEMM, RoPE/cache, flash prefill, o +
    residual, gate/up + SwiGLU, down + residual GEMMs], final-norm lm_head GEMV, greedy; the
    reference's prefill, api.cu:1807-1845), timed end to end on the host clock (it ends in a
    device->host read of the token); and the greedy decode step of B sequences at a context of ctx
    positions, captured once and replayed: up to 8 on the GEMV path (gate/up, down and lm_head on
    the GEMM where the first step times it faster), more on the GEMM path (api.cu:1914-1940)."""
    from hipinfer_amd.engine import DecodeStep
    g = torch.Generator(device="cuda")
    g.manual_seed(SEED + 21)
    embed = torch.empty(V, H, dtype=torch.float16, device="cuda").normal_(0.0, 1.0, generator=g)
    cfg = dict(H=H, Hq=HQ, Hkv=HKV, D=D, I=I, V=V, L=L, eps=1e-5, theta=500000.0)
    toks = torch.randint(0, V, (T,), generator=torch.Generator().manual_seed(SEED + 22)).tolist()
    mm_params = L * sum(N * K for N, K in SHAPES.values())
    attn_flops = L * HQ * D * 4.0 * T * (T + 1) / 2  # QK^T and PV over the causal triangle
    res = {"config": f"Llama-3.1-8B engine: prefill of a {T}-token prompt (one slot, one chunk); greedy decode "
                     f"step of B sequences at ctx {ctx} (synthetic caches, hipGraph replay): B <= 8 on the GEMV "
                     "path with the per-projection GEMM choice, larger B on the GEMM path"}
    for q8 in ([False, True] if model.q8 is not None else [False]):
        tag = "int8" if q8 else "fp16"
        W = engine_weights(model, embed, q8)
        ds = DecodeStep(cfg, W, 1, T + 16, max_prefill=T)
        ds.prefill(0, toks)  # first call: tunes the GEMM tiles of the M = T shapes
        times = []
        for _ in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            ds.prefill(0, toks)
            times.append((time.perf_counter() - t0) * 1e3)
        ms = sorted(times)[1]
        flops = 2.0 * T * mm_params + attn_flops + 2.0 * V * H
        res[f"prefill_T{T}_{tag}"] = {"ms": round(ms, 3), "tokens_per_s": round(T / ms * 1e3, 1),
                                     "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1),
                                     "pct_mfma_peak": round(100 * flops / (ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 1)}
        del ds
        torch.cuda.empty_cache()
        for B in batches:
            ds = DecodeStep(cfg, W, B, ctx + 2 * steps + 16)
            for k in ds.kc + ds.vc:
                k.normal_(0.0, 1.0, generator=g)
            ds.pos.fill_(ctx - 1)
            ds.step()  # eager: tunes the GEMM tiles (and, up to 8 sequences, the projections' paths)
            torch.cuda.synchronize()
            gr = ds.capture()
            ds.pos.fill_(ctx - 1)
            ms, _ = time_graph(torch, gr, steps, 2)
            assert torch.isfinite(ds.logits).all(), "non-finite logits (batched decode)"
            wb = weight_bytes(q8)
            kv = B * L * HKV * (ctx + steps) * D * 2 * 2
            res[f"decode_B{B}_{tag}"] = {"ms_per_step": round(ms, 4), "tokens_per_s": round(B / ms * 1e3, 1),
                                        "gemm_projections": ds.small_gemm if B > 1 and not ds.gemm_path else None,
                                        "weight_GB/s": round(wb / (ms * 1e-3) / 1e9, 1),
                                        "GB/s": round((wb + kv) / (ms * 1e-3) / 1e9, 1),
                                        "pct_hbm_peak": round(100 * (wb + kv) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1)}
            del gr, ds
            torch.cuda.empty_cache()
    del embed
    torch.cuda.empty_cache()
    return res


def prefill_bench(torch, hi, steps, warmup, q8_too):
    """Per-layer time and TFLOP/s of the four prefill GEMMs at M in {128, 512, 1024}, and of each
    GEMM kind alone at M = 1024 (the kernel the MFMA roofline is quoted on)."""
    pm = PrefillModel(torch, hi, q8_too)
    flops_layer = lambda M: 2.0 * M * sum(N * K for N, K in P_SHAPES.values())
    res = {"config": "Llama-3.2-3B prefill GEMMs (QKV 5120x3072, o 3072x3072 +res, gate/up 16384x3072 +SwiGLU, "
                     "down 3072x8192 +res), 28 distinct layers per step", "layers": {}, "kernels_m1024": {}}
    for q8 in ([False, True] if q8_too else [False]):
        tag = "int8" if q8 else "fp16"
        for M in [128, 512, 1024]:
            b = pm.buffers(M)
            g = capture(torch, lambda: pm.layer_pass(b, q8))
            ms, _ = time_graph(torch, g, max(3, steps // 2), warmup)
            us = ms * 1e3 / P_L
            # HBM bytes a layer must move at least: its weights (int8: + row scales), A in, C out
            # (and the residual read for o / down)
            wb = sum(N * K * (1 if q8 else 2) + (2 * N if q8 else 0) for N, K in P_SHAPES.values())
            ab = 2 * M * (P_SHAPES["qkv"][1] + P_SHAPES["o"][1] + P_SHAPES["gate_up"][1] + P_SHAPES["down"][1])
            cb = 2 * M * (P_SHAPES["qkv"][0] + 2 * P_SHAPES["o"][0] + P_SHAPES["gate_up"][0] // 2 + 2 * P_SHAPES["down"][0])
            hbm_us = (wb + ab + cb) / (HBM_PEAK_GBS * 1e3)
            res["layers"][f"M{M}_{tag}"] = {"us_per_layer": round(us, 2),
                                            "TFLOP/s": round(flops_layer(M) / (us * 1e-6) / 1e12, 1),
                                            "pct_mfma_peak": round(100 * flops_layer(M) / (us * 1e-6) / 1e12
                                                                   / MFMA_F16_PEAK_TFLOPS, 1),
                                            "hbm_floor_us": round(hbm_us, 2),
                                            "pct_hbm_ceiling": round(100 * hbm_us / us, 1)}
            del g
        b = pm.buffers(1024)
        # gate/up inside the layer: the layer pass minus the same pass without its gate/up launches
        # (the kernel alone, back to back, runs slower: see the roofline_mfma note)
        g = capture(torch, lambda: pm.layer_pass(b, q8, kinds=("qkv", "o", "down")))
        ms, _ = time_graph(torch, g, max(3, steps // 2), warmup)
        del g
        gu_in = res["layers"][f"M1024_{tag}"]["us_per_layer"] - ms * 1e3 / P_L
        N, K = P_SHAPES["gate_up"]
        res["gate_up_in_layer_m1024_" + tag] = {
            "us": round(gu_in, 2), "TFLOP/s": round(2.0 * 1024 * N * K / (gu_in * 1e-6) / 1e12, 1),
            "how": "M = 1024 layer pass minus the same pass without the gate/up launches (HIP events, median replays)"}
        for kind in P_SHAPES:
            g = capture(torch, lambda: pm.layer_pass(b, q8, kinds=(kind,)))
            ms, _ = time_graph(torch, g, max(3, steps // 2), warmup)
            us = ms * 1e3 / P_L
            N, K = P_SHAPES[kind]
            tf = 2.0 * 1024 * N * K / (us * 1e-6) / 1e12
            res["kernels_m1024"][f"{kind}_{tag}"] = {"N": N, "K": K, "us": round(us, 2), "TFLOP/s": round(tf, 1),
                                                     "pct_mfma_peak": round(100 * tf / MFMA_F16_PEAK_TFLOPS, 1)}
            del g
    # for scale: the vendor library (torch.matmul, hipBLASLt / rocBLAS) on the same weights at M = 1024,
    # plain GEMMs without the fused epilogues, each kind over the 28 layers in a graph
    try:
        lib = str(torch.backends.cuda.preferred_blas_library())
    except Exception:
        lib = "default"
    b = pm.buffers(1024)
    vend = {"library": "torch.matmul (" + lib + ")", "kernels_m1024": {}}
    tot = 0.0
    for kind, (N, K) in P_SHAPES.items():
        A = torch.randn(1024, K, device="cuda").half()
        outs = torch.empty(1024, N, dtype=torch.float16, device="cuda")

        def run(kind=kind, A=A, outs=outs):
            for l in range(P_L):
                torch.matmul(A, pm.layers[l][kind].t(), out=outs)
        g = capture(torch, run)
        ms, _ = time_graph(torch, g, max(3, steps // 2), warmup)
        del g
        us = ms * 1e3 / P_L
        tot += us
        tf = 2.0 * 1024 * N * K / (us * 1e-6) / 1e12
        vend["kernels_m1024"][kind] = {"us": round(us, 2), "TFLOP/s": round(tf, 1),
                                       "pct_mfma_peak": round(100 * tf / MFMA_F16_PEAK_TFLOPS, 1)}
    vend["us_per_layer_sum"] = round(tot, 2)
    vend["pct_mfma_peak"] = round(100 * flops_layer(1024) / (tot * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS, 1)
    res["vendor_m1024_fp16"] = vend
    del pm
    torch.cuda.empty_cache()
    return res


def capture(torch, fn):
    fn()  # eager warm-up: per-kernel attributes and occupancy are set outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def time_graph(torch, g, steps, warmup, full=False):
    """Replays g `steps` times after `warmup` untimed replays, with a HIP event on the replay stream
    before the first replay and after each one. Returns the median replay time in ms (the reference
    reports medians, scripts/bench.py:28-48) and the host wall time per replay; full=True adds the
    mean (first to last event over steps)."""
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    t0 = time.perf_counter()
    ev[0].record()
    for i in range(steps):
        g.replay()
        ev[i + 1].record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    med = statistics.median(ev[i].elapsed_time(ev[i + 1]) for i in range(steps))
    if full:
        return med, wall / steps, ev[0].elapsed_time(ev[steps]) / steps
    return med, wall / steps


def _cpu_layer(torch, dims, layer, q8_layer, n1, n2, seed):
    """One decode layer's weights on the host for the CPU legs: fp16 (or int8 + fp16 row scales) as
    the GPU streams them, and the fp32 copies the reference's CPU engine computes with (RefEngine
    holds fp32 weights; int8 as q * s in fp32, tests/test_kernels.py:389-390)."""
    import numpy as np
    H, Hq, Hkv, D, I = dims
    host = {k: v.cpu().numpy() for k, v in layer.items()}
    q8 = {k: (q.cpu().numpy(), s.cpu().numpy()) for k, (q, s) in q8_layer.items()}
    f32 = {k: torch.from_numpy(v.astype(np.float32)) for k, v in host.items()}
    f32q = {k: torch.from_numpy(q.astype(np.float32) * s.astype(np.float32)[:, None]) for k, (q, s) in q8.items()}
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((1, H)).astype(np.float16)
    return {"dims": dims, "fp16": host, "int8": q8, "f32": {"fp16": f32, "int8": f32q}, "x": x,
            "n1": n1.cpu().numpy(), "n2": n2.cpu().numpy()}


def _torch_layer(torch, L, fmt, eps=1e-5):
    """The reference's CPU path for one decode layer, restated in torch (scripts/ref_engine.py: mm =
    fp16(fp32 x @ W^T), 141-143; rmsnorm 145-147; swiglu / deinterleave 32-42; RoPE in fp16 ops):
    QKV (+ RoPE on q, k), o + residual (the q columns stand in for the attention output, as on the
    GPU), gate/up + SwiGLU, down + residual."""
    H, Hq, Hkv, D, I = L["dims"]
    W = L["f32"][fmt]
    r = lambda t: t.half().float()
    x = torch.from_numpy(L["x"]).float()
    n1, n2 = torch.from_numpy(L["n1"]).float(), torch.from_numpy(L["n2"]).float()
    rms = lambda v, w: r(w * r(v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + eps)))
    qkv = r(rms(x, n1) @ W["qkv"].T)
    hd = D // 2
    qk = qkv[:, :(Hq + Hkv) * D].view(1, Hq + Hkv, 2, hd)
    c, sn = torch.full((hd,), 0.6), torch.full((hd,), 0.8)
    a, b = qk[:, :, 0], qk[:, :, 1]
    rot = torch.stack([r(r(a * c) - r(b * sn)), r(r(b * c) + r(a * sn))], 2)
    q = rot.view(1, -1)[:, :Hq * D]
    x = r(x + r(q @ W["o"].T))
    gu = r(rms(x, n2) @ W["gate_up"].T).view(1, -1, 2, 16)
    g, u = gu[:, :, 0].reshape(1, I), gu[:, :, 1].reshape(1, I)
    g, u = r(g), r(u)
    act = r(r(g * torch.sigmoid(g)) * u)
    x = r(x + r(act @ W["down"].T))
    return x


def _c_layer(O, L, fmt):
    """The same layer through the C restatement (oracle/hi_oracle.c: fp64-or-better sums with the
    reference's fp16 rounding points)."""
    import numpy as np
    H, Hq, Hkv, D, I = L["dims"]
    Wd = L[fmt]
    w = (lambda k: (Wd[k], None)) if fmt == "fp16" else (lambda k: Wd[k])
    xs = L["x"].copy()
    S = 16
    hd = D // 2
    cs = np.stack([np.full((S, hd), 0.6), np.full((S, hd), 0.8)], -1).astype(np.float16)
    kc = np.zeros((1, Hkv, S, D), np.float16)
    vc = np.zeros_like(kc)
    q = np.zeros((1, Hq * D), np.float16)
    act = np.zeros((1, I), np.float16)
    Wq, sq = w("qkv")
    O.gemv_qkv_rope(xs, Wq, L["n1"], Hq, Hkv, cs, np.array([3], np.int32), kc, vc, q, scales=sq)
    Wo, so = w("o")
    O.gemv(q, Wo, out=xs, epi=1, scales=so)
    Wg, sg = w("gate_up")
    O.gemv(xs, Wg, out=act, normw=L["n2"], epi=2, scales=sg)
    Wdn, sdn = w("down")
    O.gemv(act, Wdn, out=xs, epi=1, scales=sdn)
    return xs


def _median_time(fn, runs=5, min_s=0.0):
    fn()  # warm-up (page-ins, thread pools)
    times = []
    t_end = time.perf_counter() + min_s
    while len(times) < runs or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baseline(torch, model):
    """The reference's CPU path timed on this host's cores, on the decode GEMV set of one layer of
    C2 (Llama-3.1-8B) and of C1 (TinyLlama-1.1B), fp16 and int8 weights, M = 1:
      * torch: the reference's own CPU engine restated in torch float32 (weights held in fp32, as
        RefEngine holds them; int8 as fp32 q * s), torch.get_num_threads() threads;
      * C: oracle/hi_oracle.c, the build's C restatement, with OpenMP on the job's core share and on
        one core.
    Each figure is the median of at least 5 runs; rates are the GPU format's weight bytes (what the
    GPU GEMVs stream) per second. `value` is the torch leg on C2 fp16."""
    import numpy as np

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import oracle as O

    try:
        share = len(os.sched_getaffinity(0))
    except AttributeError:
        share = os.cpu_count() or 1
    # the pool gives each one-GPU job a 16-core share (OMP_NUM_THREADS on the GPU box)
    share = max(1, min(share, int(os.environ.get("OMP_NUM_THREADS", str(share)))))
    tthreads = torch.get_num_threads()
    g = _seeded(torch, SEED + 20)
    c1_dims = (2048, 32, 4, 64, 5632)
    c1_shapes = {"qkv": ((32 + 8) * 64, 2048), "o": (2048, 2048), "gate_up": (2 * 5632, 2048), "down": (2048, 5632)}
    c1 = {k: _w(torch, g, *sh) for k, sh in c1_shapes.items()}
    c1q = {k: model.hi.quantize_rows(v) for k, v in c1.items()}
    nrm = lambda n: (torch.rand(n, generator=g, device="cuda") + 0.5).half()
    layers = {
        "C2": _cpu_layer(torch, (H, HQ, HKV, D, I), {k: model.layers[0][k] for k in SHAPES}, model.q8[0],
                         model.layers[0]["n1"], model.layers[0]["n2"], SEED + 21),
        "C1": _cpu_layer(torch, c1_dims, c1, c1q, nrm(2048), nrm(2048), SEED + 22),
    }
    legs = {}
    for name, L in layers.items():
        for fmt in ("fp16", "int8"):
            nbytes = sum(v.size * v.itemsize for v in L["fp16"].values()) if fmt == "fp16" else \
                sum(q.size + s.size * 2 for q, s in L["int8"].values())
            with torch.no_grad():
                t, n = _median_time(lambda: _torch_layer(torch, L, fmt))
            legs[f"torch_{name}_{fmt}"] = {"GB/s": round(nbytes / t / 1e9, 3), "ms": round(t * 1e3, 3),
                                           "threads": tthreads, "runs": n}
            for cores in (share, 1):
                O.set_threads(cores)
                t, n = _median_time(lambda: _c_layer(O, L, fmt))
                legs[f"c_{name}_{fmt}_{cores}core"] = {"GB/s": round(nbytes / t / 1e9, 3), "ms": round(t * 1e3, 3),
                                                       "threads": O.get_threads(), "runs": n}
    head = legs["torch_C2_fp16"]
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = None
    return {"value": head["GB/s"], "unit": "GB/s", "cores": tthreads, "kind": "port",
            "host_cpus": {"nproc": os.cpu_count(), "affinity": affinity, "job_share": share,
                          "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS")},
            "sample": "one Llama-3.1-8B layer's decode GEMVs (QKV+RoPE, o+res, gate/up+SwiGLU, down+res; "
                      "436.2 MB of fp16 weights, M = 1) through the reference's CPU engine restated in torch "
                      "float32 (scripts/ref_engine.py mm/rmsnorm/swiglu), median of >= 5 runs; legs: the same "
                      "for int8 and for a TinyLlama layer, and oracle/hi_oracle.c on %d cores and on 1 core" % share,
            "legs": legs}


# ------------------------------------------------------------------ the other BASELINE configs
def _seeded(torch, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return g


def _w(torch, g, N, K, sd=0.02):
    return torch.empty(N, K, dtype=torch.float16, device="cuda").normal_(0.0, sd, generator=g)


def _time(torch, fn, steps):
    gr = capture(torch, fn)
    ms, _ = time_graph(torch, gr, steps, 2)
    del gr
    return ms


C4_DIMS = (1536, 12, 2, 128, 8960, 151936)  # Qwen2.5-1.5B: hidden, q heads, kv heads, head dim, MLP, vocab


def decode_config_bench(torch, hi, name, dims, M_list, n_layers, steps, seed, q8_too=True, bias=False):
    """A model's decode GEMV set (QKV+RoPE, o + residual, gate/up + SwiGLU, down + residual per layer,
    then lm_head) over n_layers distinct weight sets, for each row count M: weight GB/s per token."""
    H, Hq, Hkv, D, I, V = dims
    g = _seeded(torch, seed)
    qkv_n = (Hq + 2 * Hkv) * D
    shapes = {"qkv": (qkv_n, H), "o": (H, Hq * D), "gate_up": (2 * I, H), "down": (H, I)}
    layers = [{k: _w(torch, g, *sh) for k, sh in shapes.items()} for _ in range(n_layers)]
    lm = _w(torch, g, V, H)
    qlayers = [{k: hi.quantize_rows(ly[k]) for k in shapes} for ly in layers] if q8_too else None
    lm_q = hi.quantize_rows(lm) if q8_too else None
    nw1 = (torch.rand(H, generator=g, device="cuda") + 0.5).half()
    nw2 = (torch.rand(H, generator=g, device="cuda") + 0.5).half()
    b = torch.randn(qkv_n, generator=g, device="cuda").half() if bias else None
    max_seq = 64
    ang = torch.arange(max_seq, device="cuda").float()[:, None] * (
        1.0 / 10000.0 ** (torch.arange(0, D, 2, device="cuda").float() / D))[None, :]
    cs = torch.stack([ang.cos(), ang.sin()], -1).half().contiguous()
    wbytes = lambda q8: n_layers * sum(N * K * (1 if q8 else 2) + (2 * N if q8 else 0) for N, K in shapes.values()) + \
        V * H * (1 if q8 else 2) + (2 * V if q8 else 0)
    out = {"shapes": {k: list(v) for k, v in shapes.items()}, "lm_head": [V, H], "layers": n_layers, "tokens": {}}
    for M in M_list:
        kc = torch.zeros(M, Hkv, max_seq, D, dtype=torch.float16, device="cuda")
        vc = torch.zeros_like(kc)
        pos = torch.full((M,), 5, dtype=torch.int32, device="cuda")
        x0 = torch.randn(M, H, generator=g, device="cuda").half()
        x = x0.clone()
        q = torch.empty(M, Hq * D, dtype=torch.float16, device="cuda")
        act = torch.empty(M, I, dtype=torch.float16, device="cuda")
        logits = torch.empty(M, V, dtype=torch.float16, device="cuda")
        for q8 in ([False, True] if q8_too else [False]):
            def token():
                x.copy_(x0)
                for l in range(n_layers):
                    wsrc = qlayers[l] if q8 else {k: (layers[l][k], None) for k in shapes}
                    W, sc = wsrc["qkv"]
                    hi.gemv_qkv_rope(x, W, nw1, Hq, Hkv, cs, pos, kc, vc, q, bias=b, scales=sc)
                    W, sc = wsrc["o"]
                    hi.gemv(q, W, out=x, epi=1, scales=sc)
                    W, sc = wsrc["gate_up"]
                    hi.gemv(x, W, out=act, normw=nw2, epi=2, scales=sc)
                    W, sc = wsrc["down"]
                    hi.gemv(act, W, out=x, epi=1, scales=sc)
                W, sc = (lm_q if q8 else (lm, None))
                hi.gemv(x, W, out=logits, normw=nw1, scales=sc)
            ms = _time(torch, token, steps)
            wb = wbytes(q8)
            out["tokens"][f"M{M}_{'int8' if q8 else 'fp16'}"] = {
                "ms_per_token_set": round(ms, 4), "weight_GB/s": round(wb / (ms * 1e-3) / 1e9, 1),
                "pct_hbm_peak": round(100 * wb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1), "weight_bytes": wb}
    del layers, qlayers, lm, lm_q
    torch.cuda.empty_cache()
    out["config"] = name
    return out


def moe_bench(torch, hi, steps, seed):
    """Granite-3.1-1B-A400M-shaped MoE layers (hidden 1024, 32 experts of SwiGLU 1024 -> 2 x 512 and
    512 -> 1024, top-8, softmax over the top-8 logits, fp16 routing weights, residual scale 0.22) over
    24 distinct layers: B = 1 decode as the reference's two calls (router, then GEMV experts) and as
    this library's one call (one launch), and a 256-token prefill as the reference's two calls
    (router, then the grouped MFMA experts: sort, two GEMMs, combine) and as the one call (the sort
    inside the router's launch)."""
    H, E, I, k, L = 1024, 32, 512, 8, 24
    flags = hi.MOE_NORM_TOPK | hi.MOE_FP16_WEIGHTS
    g = _seeded(torch, seed)
    Wr = [_w(torch, g, E, H) for _ in range(L)]
    wgu = [torch.empty(E, 2 * I, H, dtype=torch.float16, device="cuda").normal_(0, 0.02, generator=g) for _ in range(L)]
    wdn = [torch.empty(E, H, I, dtype=torch.float16, device="cuda").normal_(0, 0.02, generator=g) for _ in range(L)]
    res = {"config": "Granite-3.1-1B-A400M MoE layer: H 1024, 32 experts (gate/up 1024->2x512, down 512->1024), "
                     "top-8, 24 distinct layers per step"}
    for M, path, tag in [(1, 1, "decode_B1_gemv"), (1, -1, "decode_B1_fused"), (256, 2, "prefill_256_grouped"),
                         (256, -1, "prefill_256_fused")]:
        xn = torch.randn(M, H, generator=g, device="cuda").half()
        x0 = torch.randn(M, H, generator=g, device="cuda").half()
        x = x0.clone()
        work = torch.zeros(hi.lib.hi_moe_work_bytes(M, k, E, H, I), dtype=torch.uint8, device="cuda")
        idx = torch.empty(M, k, dtype=torch.int32, device="cuda")
        wts = torch.empty(M, k, dtype=torch.float32, device="cuda")

        def step():
            x.copy_(x0)
            for l in range(L):
                if path < 0:  # router + experts in one call
                    hi.lib.hi_moe_route_experts(hi.ptr(xn), xn.stride(0), hi.ptr(Wr[l]), hi.ptr(wgu[l]), hi.ptr(wdn[l]), M,
                                                E, k, H, I, flags, 0.22, hi.ptr(x), x.stride(0), hi.ptr(idx),
                                                hi.ptr(wts), hi.ptr(work), hi.cur_stream())
                    continue
                hi.lib.hi_moe_router(hi.ptr(xn), xn.stride(0), hi.ptr(Wr[l]), M, E, H, k, flags, hi.ptr(idx), hi.ptr(wts),
                                     hi.cur_stream())
                hi.lib.hi_moe_experts(hi.ptr(xn), xn.stride(0), hi.ptr(wgu[l]), hi.ptr(wdn[l]), hi.ptr(idx), hi.ptr(wts), M,
                                      E, k, H, I, flags, 0.22, hi.ptr(x), x.stride(0), path, hi.ptr(work), hi.cur_stream())
        ms = _time(torch, step, steps)
        us = ms * 1e3 / L
        if M == 1:
            used = idx.unique().numel()
            b = E * H * 2 + used * (2 * I * H + H * I) * 2
            res[tag] = {"us_per_layer": round(us, 2), "experts_read": used, "bytes_per_layer": b,
                        "GB/s": round(b / us / 1e3, 1), "pct_hbm_peak": round(100 * b / us / 1e3 / HBM_PEAK_GBS, 1)}
        else:
            flops = 2.0 * M * k * (2 * I * H + H * I) + 2.0 * M * E * H
            # every expert's weights and the router once, xn read, x read and written, the pairs'
            # activations (I) and down outputs (H) written and read once each
            b = E * (2 * I * H + H * I) * 2 + E * H * 2 + 3 * M * H * 2 + 2 * M * k * (I + H) * 2
            res[tag] = {"us_per_layer": round(us, 2), "TFLOP/s": round(flops / (us * 1e-6) / 1e12, 1),
                        "expert_pairs": M * k, "bytes_per_layer": b, "GB/s": round(b / us / 1e3, 1),
                        "pct_hbm_peak": round(100 * b / us / 1e3 / HBM_PEAK_GBS, 1)}
    del Wr, wgu, wdn
    torch.cuda.empty_cache()
    return res


def traffic_from_profile():
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3 --pmc summary
    (FETCH_SIZE and WRITE_SIZE runs, each scaled by the same counter's reading for a plain copy of
    known size). None when the summary is absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "gemv_gate_up_llama31_8b_hbm_bytes.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1].strip())
    except OSError:
        pass
    return None


def copy_bandwidth(torch, nbytes=1 << 30, reps=10):
    """A plain device-to-device copy of nbytes (torch's copy kernel), timed with HIP events: bytes
    read plus bytes written per second, the practical HBM rate next to the 8 TB/s datasheet figure."""
    src = torch.empty(nbytes // 2, dtype=torch.float16, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    del src, dst
    torch.cuda.empty_cache()
    return {"GB/s": round(2 * nbytes / us / 1e3, 1), "bytes_moved": 2 * nbytes, "us": round(us, 2),
            "pct_hbm_peak": round(100 * 2 * nbytes / us / 1e3 / HBM_PEAK_GBS, 1)}


def prefill_breakdown(csv_path):
    """Per-kernel time of the last engine prefill (or decode step) in a rocprofv3 kernel trace
    (`--kernel-trace --output-format csv`) of `bench.py --profile prefill` (or `decode64`): the
    launches after the second-to-last greedy argmax up to the last one (one whole prefill or
    step: embed, 32 layers, lm_head, argmax). Prints a markdown table, longest total first."""
    import csv
    with open(csv_path) as f:
        rows = sorted(((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"])
                       for r in csv.DictReader(f)), key=lambda t: t[0])
    ends = [i for i, r in enumerate(rows) if "argmax" in r[2]]
    seg = rows[ends[-2] + 1:ends[-1] + 1]
    span = (seg[-1][1] - seg[0][0]) / 1e3
    agg = {}
    for start, end, name in seg:
        d = agg.setdefault(name.split("(")[0], [0, 0.0])
        d[0] += 1
        d[1] += (end - start) / 1e3
    busy = sum(v[1] for v in agg.values())
    print(f"span (first launch start to last launch end): {span:.1f} us; kernels busy {busy:.1f} us; "
          f"{len(seg)} launches")
    print("| kernel | launches | avg us | total us | share of busy |")
    print("|---|---|---|---|---|")
    for name, (c, t) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        print(f"| `{name[:80]}` | {c} | {t / c:.2f} | {t:.1f} | {100 * t / busy:.1f} % |")


def timeline(csv_path):
    """Per-kind durations and launch gaps of replayed decode tokens, from a rocprofv3 kernel trace
    (`--kernel-trace --output-format csv`) of `bench.py --profile token` / `token8`. A token is the
    run of 129 GEMV launches (32 x [QKV, o, gate/up, down] + lm_head); each GEMV is named by its
    epilogue (template argument 3: 3 QKV+RoPE, 1 residual, 2 SwiGLU, 0 lm_head), and the residual
    launch after QKV is o, after gate/up down. The gap of a launch is the time from the previous
    launch's end to its start. Prints a markdown table."""
    import csv
    import re
    rows = []
    with open(csv_path) as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"]
            m = re.search(r"gemv\w*<\s*(\d+),\s*(true|false),\s*(\d+)", name)
            if m:
                rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), int(m.group(3))))
    rows.sort()
    per_token = 32 * 4 + 1
    tokens = [rows[i:i + per_token] for i in range(0, len(rows) - per_token + 1, per_token)]
    tokens = [t for t in tokens if [e for _, _, e in t[:4]] == [3, 1, 2, 1] and t[-1][2] == 0]
    tokens = tokens[2:] if len(tokens) > 3 else tokens  # skip the eager pass and the first replay
    stats = {}
    spans = []
    for t in tokens:
        spans.append((t[-1][1] - t[0][0]) / 1e3)
        prev_end, prev_kind = None, None
        for start, end, epi in t:
            kind = {3: "qkv", 2: "gate_up", 0: "lm_head"}.get(epi) or ("o" if prev_kind == "qkv" else "down")
            d = stats.setdefault(kind, [0, 0.0, 0.0, 0])  # launches, busy us, gap us, gaps measured
            d[0] += 1
            d[1] += (end - start) / 1e3
            if prev_end is not None:  # a token's first launch has no launch before it in the token
                d[2] += (start - prev_end) / 1e3
                d[3] += 1
            prev_end, prev_kind = end, kind
    n = len(tokens)
    print(f"tokens analysed: {n}; token span (first launch start to last launch end): "
          f"{sum(spans) / n:.1f} us (min {min(spans):.1f}, max {max(spans):.1f})")
    print("| kind | launches per token | avg duration us | avg gap before us | per token: busy us | gaps us |")
    print("|---|---|---|---|---|---|")
    tb = tg = 0.0
    for kind in ["qkv", "o", "gate_up", "down", "lm_head"]:
        c, dur, gap, ng = stats[kind]
        per = c // n
        tb += dur / n
        tg += gap / n
        print(f"| {kind} | {per} | {dur / c:.2f} | {gap / max(1, ng):.2f} | {dur / n:.1f} | {gap / n:.1f} |")
    print(f"| all | {per_token} | | | {tb:.1f} | {tg:.1f} |")


def gemm_counters(csv_paths, cus=256, xcds=8, replays=3):
    """Per-GEMM-kind counters of the last `replays` layer passes of `bench.py --profile gemm`, from one
    or more rocprofv3 `--pmc` counter CSVs of that command (one counter pass each; every pass also
    collects GRBM_GUI_ACTIVE). A pass is 28 layers x (QKV, o, gate/up, down) GEMM launches, in that
    order, so a launch's kind is its position. Prints up to two markdown tables:
      * MfmaUtil = 100 * SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE * CUs * 4), rocprofv3's own
        derived metric, with GRBM_GUI_ACTIVE taken per XCD (the raw counter is the sum of the 8 XCDs'
        copies), the MFMA flop count (SQ_INSTS_VALU_MFMA_MOPS_F16 x 512) and SQ_WAIT_INST_ANY;
      * the memory path (when its counters were collected): LDS indexed-access cycles, bank and
        address conflict cycles, TA busy, TD busy and TD stalled on the TC, TCP tag lookups, tag
        conflicts and waits for L2 data, each per CU per GPU-active cycle."""
    import csv
    kinds = ["qkv", "o", "gate_up", "down"]
    agg = {k: {"n": {}} for k in kinds}
    total = 0
    passes = {}  # path -> the counters it collected
    for path in ([csv_paths] if isinstance(csv_paths, str) else csv_paths):
        disp = {}
        with open(path) as f:
            for r in csv.DictReader(f):
                if "gemm_kernel" not in r["Kernel_Name"]:
                    continue
                d = disp.setdefault(int(r["Dispatch_Id"]), {"name": r["Kernel_Name"]})
                d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
                passes.setdefault(path, set()).add(r["Counter_Name"])
        ids = sorted(disp)
        total = len(ids)
        last = ids[-replays * P_L * 4:]
        for i, d_id in enumerate(last):
            a = agg[kinds[i % 4]]
            a["name"] = disp[d_id]["name"]
            for c, v in disp[d_id].items():
                if c == "name":
                    continue
                if c == "GRBM_GUI_ACTIVE":  # the same per pass: keep one pass's
                    c = "GRBM_GUI_ACTIVE@" + path
                a[c] = a.get(c, 0.0) + v
                a["n"][c] = a["n"].get(c, 0) + 1

    def active(a, counter):
        # GPU-active cycles (per XCD) summed over the kind's launches, from the pass that has `counter`
        for c in a:
            if c.startswith("GRBM_GUI_ACTIVE@") and counter in passes.get(c.split("@", 1)[1], ()):
                return a[c] / xcds
        return max(1.0, next((a[c] for c in a if c.startswith("GRBM_GUI_ACTIVE@")), 1.0) / xcds)

    print(f"dispatches: {total} gemm_kernel launches in the trace; the last {replays * P_L * 4} ({replays} passes) used")
    if any("SQ_VALU_MFMA_BUSY_CYCLES" in agg[k] for k in kinds):
        print("| GEMM | kernel | MfmaUtil % | MFMA flop per launch (MOPs x 512) | SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES % "
              "| GPU-active cycles per launch (per XCD) |")
        print("|---|---|---|---|---|---|")
        for k in kinds:
            a = agg[k]
            act = active(a, "SQ_VALU_MFMA_BUSY_CYCLES")
            n = max(1, a["n"].get("SQ_VALU_MFMA_BUSY_CYCLES", 1))
            util = 100 * a.get("SQ_VALU_MFMA_BUSY_CYCLES", 0) / max(1.0, act * cus * 4)
            wait = 100 * a.get("SQ_WAIT_INST_ANY", 0) / max(1.0, a.get("SQ_WAVE_CYCLES", 0))
            name = a.get("name", "")
            name = name[name.find("gemm_kernel"):][:60]
            mops = a.get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0) * 512 / n
            print(f"| {k} | `{name}` | {util:.1f} | {mops:.4g} | {wait:.1f} | {act / n:.0f} |")
    mem = ["SQ_LDS_IDX_ACTIVE", "SQ_LDS_BANK_CONFLICT", "SQ_LDS_ADDR_CONFLICT", "TA_BUSY_avr", "TD_TD_BUSY_sum",
           "TD_TC_STALL_sum", "TCP_TOTAL_CACHE_ACCESSES_sum", "TCP_READ_TAGCONFLICT_STALL_CYCLES_sum",
           "TCP_PENDING_STALL_CYCLES_sum"]
    have = [c for c in mem if any(c in agg[k] for k in kinds)]
    if have:
        print()
        print("| GEMM | " + " | ".join(have) + " |")
        print("|---|" + "---|" * len(have))
        for k in kinds:
            a = agg[k]
            row = []
            for c in have:
                act = active(a, c)
                # TA_BUSY_avr is an average over the TA instances (one per CU): per GPU-active cycle;
                # the others are sums over CUs: per CU per GPU-active cycle
                v = a.get(c, 0.0) / max(1.0, act if c == "TA_BUSY_avr" else act * cus)
                row.append(f"{v:.3f}")
            print(f"| {k} | " + " | ".join(row) + " |")


def gemm_clock(trace_csv, counter_csv, replays, xcds=8):
    """Shader clock of the M = 1024 gate/up GEMM inside the layer and back to back, from two runs of
    `bench.py --profile gemm_clock --steps <replays>`: a rocprofv3 --kernel-trace run (durations) and a
    --pmc GRBM_GUI_ACTIVE run (GPU-active cycles, the raw counter summed over the XCDs' copies). The
    profile ends with `replays` layer passes (28 x QKV, o, gate/up, down) and then `replays` passes of
    the 28 gate/up launches alone (each preceded by one eager pass); the gate/up launch is every
    fourth GEMM of a layer pass. Prints duration, cycles and cycles per microsecond (MHz) per mode."""
    import csv
    trace = []
    with open(trace_csv) as f:
        for r in csv.DictReader(f):
            if "gemm_kernel" in r["Kernel_Name"]:
                trace.append((int(r["Dispatch_Id"]), (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3))
    trace.sort()
    cyc, cdur = {}, {}
    with open(counter_csv) as f:
        for r in csv.DictReader(f):
            if "gemm_kernel" in r["Kernel_Name"] and r["Counter_Name"] == "GRBM_GUI_ACTIVE":
                k = int(r["Dispatch_Id"])
                cyc[k] = cyc.get(k, 0.0) + float(r["Counter_Value"])
                cdur[k] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    cycles = [cyc[k] / xcds for k in sorted(cyc)]
    cdurs = [cdur[k] for k in sorted(cyc)]
    n_gu, n_layer = replays * P_L, replays * P_L * 4
    durs = [d for _, d in trace]
    lay = slice(-n_gu - P_L - n_layer, -n_gu - P_L)
    modes = {"back to back (28 gate/up launches per pass)": (durs[-n_gu:], cycles[-n_gu:], cdurs[-n_gu:]),
             "inside the layer pass (every 4th GEMM)": (durs[lay][2::4], cycles[lay][2::4], cdurs[lay][2::4])}
    print("| gate/up (M = 1024) | launches | mean us (trace run) | mean us (counter run) | GPU-active cycles per "
          "launch (per XCD) | cycles per us of the counter run |")
    print("|---|---|---|---|---|---|")
    for name, (d, c, cd) in modes.items():
        md, mc, mcd = sum(d) / len(d), sum(c) / len(c), sum(cd) / len(cd)
        print(f"| {name} | {len(d)} | {md:.2f} | {mcd:.2f} | {mc:.0f} | {mc / mcd:.0f} |")


def gemv_counters(csv_paths, layers=28, cus=256, clock_ghz=2.4):
    """Per-kind counters of a decode GEMV set, from one or more rocprofv3 `--pmc` counter CSVs of the same
    command (one counter pass each): `bench.py --profile c4` (the C4 set at 5 and 8 rows, 28 layers, each
    row count fp16 tokens then int8 tokens) or `bench.py --profile tokens` (the C2 set at one row, 32
    layers, fp16 tokens then int8 tokens). A token is `layers` x (QKV, o, gate/up, down) + lm_head GEMV
    launches in that order, so a launch's kind is its position in its token; o and down share one kernel
    instance and are told apart this way. Sums every token's launches per (kind, format, rows). Columns:
      * waves per launch (SQ_WAVES), VALU and LDS instructions per wave;
      * the launch's duration in the counter run (its dispatch timestamps);
      * the SIMDs' VALU share: SQ_ACTIVE_INST_VALU (in 4-cycle units, one per wave64 VALU instruction)
        spread over the CUs' 4 SIMDs, at `clock_ghz`, against that duration;
      * resident waves per SIMD, SQ_WAVE_CYCLES (4-cycle units) spread the same way: the mean over the
        launch, below the occupancy limit while the waves ramp up and drain;
      * VALU-active, SQ_WAIT_INST_ANY and LDS-wait cycles as shares of each wave's own cycles;
      * FETCH_SIZE per launch (when that pass was collected) in MB, scaled by what the counter reads for
        the profile's closing 1 GiB device copy (1,073,741,824 bytes read), or by 2.0, the factor the
        same calibration gave on MI355X, when the run has no such copy."""
    import csv
    kinds = ["qkv", "o", "gate_up", "down"]
    per_token = layers * 4 + 1
    agg = {}
    copies = []  # FETCH_SIZE readings (KiB) of the 1 GiB calibration copy
    for path in csv_paths:
        disp = {}
        with open(path) as f:
            for r in csv.DictReader(f):
                if "copyBuffer" in r["Kernel_Name"] and r["Counter_Name"] == "FETCH_SIZE" and \
                        float(r["Counter_Value"]) > 2 ** 18:
                    copies.append(float(r["Counter_Value"]))
                if "gemv_kernel" not in r["Kernel_Name"]:
                    continue
                d = disp.setdefault(int(r["Dispatch_Id"]), {"name": r["Kernel_Name"]})
                d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
                d["us"] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        for i, d_id in enumerate(sorted(disp)):
            d = disp[d_id]
            j = i % per_token
            kind = "lm_head" if j == per_token - 1 else kinds[j % 4]
            # the rows and the format are the kernel's MR and WF template arguments: <MR, NORM, EPI, WF, G>
            args = d["name"][d["name"].find("<") + 1:d["name"].find(">")].split(",")
            mr = int(args[0])
            fmt = "int8" if args[3].strip() != "0" else "fp16"
            a = agg.setdefault((kind, fmt, mr), {"name": d["name"], "n": {}})
            for c, v in d.items():
                if c == "name":
                    continue
                if c == "us":  # the duration, per pass (one pass's counters go with its own durations)
                    c = "us@" + path
                a[c] = a.get(c, 0.0) + v
                a["n"][c] = a["n"].get(c, 0) + 1

    def us(a, counter):  # summed durations of the kind's launches in the pass that collected `counter`
        for c in a:
            if c.startswith("us@") and counter in a and a["n"].get(counter) == a["n"][c]:
                return a[c]
        return 0.0

    simds = cus * 4
    per_us = clock_ghz * 1e3 / 4  # 4-cycle units per microsecond
    scale = 2 ** 20 / (sum(copies) / len(copies)) if copies else 2.0  # bytes per KiB of FETCH_SIZE / 1024
    print(f"FETCH_SIZE scale: {scale:.4f} ({'from the 1 GiB copy in this run' if copies else 'no calibration copy in this run: the MI355X factor'})")
    print()
    print("| kind | format | rows | kernel | launches | waves per launch | duration us | VALU instructions per wave "
          "| SIMD VALU share % | resident waves per SIMD | VALU-active / wave cycles % "
          "| SQ_WAIT_INST_ANY / wave cycles % | LDS instructions per wave | LDS wait / wave cycles % "
          "| HBM reads per launch MB (FETCH_SIZE, scaled) |")
    print("|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|")
    for mr in sorted({k[2] for k in agg}):
        for fmt in ("fp16", "int8"):
            for kind in kinds + ["lm_head"]:
                a = agg.get((kind, fmt, mr))
                if not a:
                    continue
                w, wc = a.get("SQ_WAVES", 0), a.get("SQ_WAVE_CYCLES", 0)
                n = max(a["n"].get("SQ_WAVES", 0), a["n"].get("FETCH_SIZE", 0))
                nw = max(1, a["n"].get("SQ_WAVES", 1))
                name = a["name"][a["name"].find("gemv_kernel"):a["name"].find(">") + 1]
                fetch = a.get("FETCH_SIZE", 0) / max(1, a["n"].get("FETCH_SIZE", 1)) * 1024 * scale / 1e6
                t_v, t_w = us(a, "SQ_ACTIVE_INST_VALU"), us(a, "SQ_WAVE_CYCLES")
                share = f"{100 * a.get('SQ_ACTIVE_INST_VALU', 0) / simds / per_us / t_v:.1f}" if t_v else "-"
                res = f"{wc / simds / per_us / t_w:.2f}" if t_w else "-"
                dur = f"{t_v / nw:.2f}" if t_v else "-"
                print(f"| {kind} | {fmt} | {mr} | `{name}` | {n} | {w / nw:.0f} | {dur} | "
                      f"{a.get('SQ_INSTS_VALU', 0) / max(1, w):.0f} | {share} | {res} | "
                      f"{100 * a.get('SQ_ACTIVE_INST_VALU', 0) / max(1, wc):.1f} | "
                      f"{100 * a.get('SQ_WAIT_INST_ANY', 0) / max(1, wc):.1f} | {a.get('SQ_INSTS_LDS', 0) / max(1, w):.0f} | "
                      f"{100 * a.get('SQ_WAIT_INST_LDS', 0) / max(1, wc):.1f} | {fetch:.2f} |")


def main():
    if len(sys.argv) >= 3 and sys.argv[1] == "--gemv-counters":
        if sys.argv[2] == "--layers":  # --gemv-counters --layers 32 <csv>... for --profile tokens
            gemv_counters(sys.argv[4:], layers=int(sys.argv[3]))
        else:
            gemv_counters(sys.argv[2:])
        return
    if len(sys.argv) == 3 and sys.argv[1] == "--timeline":
        timeline(sys.argv[2])
        return
    if len(sys.argv) == 5 and sys.argv[1] == "--gemm-clock":
        gemm_clock(sys.argv[2], sys.argv[3], int(sys.argv[4]))
        return
    if len(sys.argv) >= 3 and sys.argv[1] == "--gemm-counters":
        gemm_counters(sys.argv[2:])
        return
    if len(sys.argv) == 3 and sys.argv[1] == "--prefill-breakdown":
        prefill_breakdown(sys.argv[2])
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-int8", action="store_true")
    ap.add_argument("--no-gemm", action="store_true", help="skip the prefill GEMM (C3) section")
    ap.add_argument("--no-configs", action="store_true", help="skip the C1 / C4 / C5 sections")
    ap.add_argument("--no-step", action="store_true", help="skip the whole decode step (with attention) section")
    ap.add_argument("--no-engine", action="store_true", help="skip the engine prefill / batched decode section")
    ap.add_argument("--prefill-breakdown", metavar="CSV", default=None,
                    help="(alone) print the per-kernel table of the last prefill (or decode step) in a kernel "
                         "trace of --profile prefill (or decode64)")
    ap.add_argument("--profile", choices=["token", "token8", "tokens", "gemm", "gemm_clock", "moe", "c4", "prefill",
                                          "flash", "decode64"] +
                    [k + q for k in ("qkv", "o", "gate_up", "down", "lm_head") for q in ("", "8")], default=None,
                    help="only run the named GEMV set (for rocprofv3 counter runs), then exit")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (the matmul hot path on one MI355X); "
              f"--gpus {args.gpus} / WORLD_SIZE {world} is not supported", file=sys.stderr)
        sys.exit(2)

    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from hipinfer_amd import hipinfer as hi

    assert torch.cuda.is_available(), "bench.py needs the GPU"
    log(f"device: {torch.cuda.get_device_name(0)}, {hi.lib.hi_device_cus()} CUs")
    if args.profile == "moe":
        log(json.dumps(moe_bench(torch, hi, args.steps, SEED + 12)))
        return
    if args.profile == "flash":  # flash prefill alone, Llama-3.1-8B heads, T = 1024 / 2048 / 4096, 10 launches each
        g = torch.Generator(device="cuda")
        g.manual_seed(SEED + 23)
        for T in (1024, 2048, 4096):
            kc = torch.empty(HKV, T, D, dtype=torch.float16, device="cuda").normal_(generator=g)
            vc = torch.empty(HKV, T, D, dtype=torch.float16, device="cuda").normal_(generator=g)
            qq = torch.empty(T, HQ * D, dtype=torch.float16, device="cuda").normal_(generator=g)
            oo = torch.empty_like(qq)
            for _ in range(10):
                hi.flash_prefill(qq, kc, vc, T, 0, HQ, HKV, out=oo)
            torch.cuda.synchronize()
        log("profile run done (flash)")
        return
    if args.profile == "decode64":  # engine decode step of 64 sequences at 1024 positions, fp16, graph replays
        model = Model(torch, hi, q8_too=False)
        from hipinfer_amd.engine import DecodeStep
        g = torch.Generator(device="cuda")
        g.manual_seed(SEED + 21)
        embed = torch.empty(V, H, dtype=torch.float16, device="cuda").normal_(0.0, 1.0, generator=g)
        cfg = dict(H=H, Hq=HQ, Hkv=HKV, D=D, I=I, V=V, L=L, eps=1e-5, theta=500000.0)
        ds = DecodeStep(cfg, engine_weights(model, embed, False), 64, 1024 + 64)
        for k in ds.kc + ds.vc:
            k.normal_(0.0, 1.0, generator=g)
        ds.pos.fill_(1023)
        ds.step()  # eager: tunes the GEMM tiles
        torch.cuda.synchronize()
        gr = ds.capture()
        ds.pos.fill_(1023)
        for _ in range(5):
            gr.replay()
        torch.cuda.synchronize()
        log("profile run done (decode64)")
        return
    if args.profile == "prefill":  # engine prefill of a 1024-token prompt, fp16: a tuning call, then 3
        model = Model(torch, hi, q8_too=False)
        from hipinfer_amd.engine import DecodeStep
        g = torch.Generator(device="cuda")
        g.manual_seed(SEED + 21)
        embed = torch.empty(V, H, dtype=torch.float16, device="cuda").normal_(0.0, 1.0, generator=g)
        cfg = dict(H=H, Hq=HQ, Hkv=HKV, D=D, I=I, V=V, L=L, eps=1e-5, theta=500000.0)
        toks = torch.randint(0, V, (1024,), generator=torch.Generator().manual_seed(SEED + 22)).tolist()
        ds = DecodeStep(cfg, engine_weights(model, embed, False), 1, 1024 + 16, max_prefill=1024)
        for _ in range(4):
            ds.prefill(0, toks)
        torch.cuda.synchronize()
        log("profile run done (prefill)")
        return
    if args.profile == "c4":  # the C4 GEMV set at 5 and 8 rows (speculative-verify widths), fp16 then int8 each
        log(json.dumps(decode_config_bench(torch, hi, "C4 at 5 and 8 rows", C4_DIMS, [5, 8], 28, args.steps,
                                           SEED + 11, bias=True)))
        return
    t0 = time.perf_counter()
    model = Model(torch, hi, q8_too=not args.no_int8)
    log(f"weights ready in {time.perf_counter() - t0:.1f} s")

    if args.profile:
        if args.profile == "gemm_clock":
            # the M = 1024 layer pass, then the gate/up launches alone back to back: `steps` replays of
            # each, for the shader-clock comparison (--gemm-clock)
            pm = PrefillModel(torch, hi, False)
            b = pm.buffers(1024)
            for kinds in [("qkv", "o", "gate_up", "down"), ("gate_up",)]:
                g = capture(torch, lambda: pm.layer_pass(b, False, kinds=kinds))
                for _ in range(args.steps):
                    g.replay()
                torch.cuda.synchronize()
                del g
            log(f"profile run done (gemm_clock): {args.steps} layer passes, then {args.steps} gate/up passes")
            return
        if args.profile == "gemm":
            pm = PrefillModel(torch, hi, False)
            b = pm.buffers(1024)
            fns = [lambda: pm.layer_pass(b, False)]
        elif args.profile == "tokens":  # the fp16 token, then the int8 token (--gemv-counters --layers 32)
            fns = [lambda: model.token(False), lambda: model.token(True)]
        else:
            q8 = args.profile.endswith("8")
            kind = args.profile.rstrip("8")
            fns = [(lambda: model.token(q8)) if kind == "token" else (lambda: model.one_kind(kind, q8))]
        for fn in fns:
            g = capture(torch, fn)
            for _ in range(args.steps):
                g.replay()
            torch.cuda.synchronize()
            del g
        # a plain device copy of known size, to calibrate the HBM byte counters
        src = torch.empty(1 << 29, dtype=torch.float16, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"profile run done ({args.profile}); copy kernel moved {src.numel() * 2} bytes each way x3")
        return

    # ---- the step: one fp16 token through all 32 layers + lm_head
    g16 = capture(torch, lambda: model.token(False))
    ms16, wall16, mean16 = time_graph(torch, g16, args.steps, args.warmup, full=True)
    assert torch.isfinite(model.logits).all(), "non-finite logits"
    out = {"fp16": (ms16, wall16, mean16)}
    kernels = {}
    if model.q8 is not None:
        g8 = capture(torch, lambda: model.token(True))
        ms8, wall8, mean8 = time_graph(torch, g8, args.steps, args.warmup, full=True)
        assert torch.isfinite(model.logits).all(), "non-finite logits (int8)"
        out["int8"] = (ms8, wall8, mean8)
    # ---- each GEMV kind alone (32 distinct weight sets back to back), fp16 and int8
    for q8 in ([False, True] if model.q8 is not None else [False]):
        for kind in ["qkv", "o", "gate_up", "down", "lm_head"]:
            n = [0]

            def fn(kind=kind, q8=q8):
                n[0] = model.one_kind(kind, q8)
            g = capture(torch, fn)
            ms, _ = time_graph(torch, g, max(3, args.steps // 2), 2)
            N, K = SHAPES[kind] if kind != "lm_head" else (V, H)
            b = N * K * (1 if q8 else 2) + (2 * N if q8 else 0)
            us = ms * 1e3 / n[0]
            kernels[f"{kind}_{'int8' if q8 else 'fp16'}"] = {
                "N": N, "K": K, "us": round(us, 2), "GB/s": round(b / us / 1e3, 1),
                "pct_hbm_peak": round(100 * b / us / 1e3 / HBM_PEAK_GBS, 1)}
    gu = kernels["gate_up_fp16"]
    N, K = SHAPES["gate_up"]
    alg = N * K * 2 + (H * 2 + (N // 2) * 2 + H * 2)  # weights + x + out + norm weight
    roofline = {"bound": "hbm", "achieved": round(alg / gu["us"] / 1e3, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(alg / gu["us"] / 1e3 / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": "gemv_kernel<MR=1,NORM,EPI=2 (SwiGLU),fp16> gate/up 28672x4096",
                "launch_bytes": alg, "avg_us": gu["us"]}

    wb16 = weight_bytes(False)
    value = wb16 / (ms16 * 1e-3) / 1e9
    res = {
        "metric": "decode GEMV GB/s (% HBM peak) + prefill GEMM TFLOP/s, 8B shapes fp16/int8",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms16, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic (seeded N(0,0.02) weights of the architecture, generated on the GPU)",
        "config": {"workload": "Llama-3.1-8B decode GEMV set, batch 1: 32 layers x (QKV+RoPE, o, gate/up, down) + "
                               "lm_head, every weight streamed once per token (hipGraph replay)",
                   "weight_bytes_per_step": wb16, "act_bytes_per_step": act_bytes()},
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "timing": "ms_per_step is the median replay (HIP events around each replay); mean over all steps beside it",
        "mean_ms_per_step": round(mean16, 4),
        "wall_ms_per_step": round(wall16, 4),
    }
    if "int8" in out:
        wb8 = weight_bytes(True)
        v8 = wb8 / (out["int8"][0] * 1e-3) / 1e9
        res["int8"] = {"value": round(v8, 1), "unit": "GB/s", "ms_per_step": round(out["int8"][0], 4),
                       "mean_ms_per_step": round(out["int8"][2], 4),
                       "pct_hbm_peak": round(100 * v8 / HBM_PEAK_GBS, 2), "weight_bytes_per_step": wb8}
    res["kernels"] = kernels
    roofline["traffic"] = traffic_from_profile()
    roofline["traffic_source"] = "profiles/gemv_gate_up_llama31_8b_hbm_bytes.md (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)"
    res["roofline"] = roofline
    if not args.no_step:
        log("decode step ...")
        res["decode_step"] = decode_step_bench(torch, hi, model, args.steps)
    if not args.no_engine:
        log("engine prefill / batched decode ...")
        res["engine"] = engine_bench(torch, hi, model, args.steps)
    if not args.no_gemm:
        log("prefill GEMM ...")
        res["prefill_gemm"] = prefill_bench(torch, hi, args.steps, args.warmup, not args.no_int8)
        gk = res["prefill_gemm"]["kernels_m1024"]["gate_up_fp16"]
        gi = res["prefill_gemm"]["gate_up_in_layer_m1024_fp16"]
        flops = 2.0 * 1024 * gk["N"] * gk["K"]
        res["roofline_mfma"] = {
            "bound": "mfma", "achieved": gk["TFLOP/s"], "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(gk["TFLOP/s"] / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None,
            "kernel": "gemm_kernel (tuned tile) gate/up + SwiGLU, Llama-3.2-3B, M=1024, N=16384, K=3072, fp16",
            "launch_flops": flops, "avg_us": gk["us"],
            "avg_us_how": "28 distinct gate/up launches back to back in a graph (HIP events, median replay / 28)",
            "in_layer_us": gi["us"], "in_layer_frac": round(gi["TFLOP/s"] / MFMA_F16_PEAK_TFLOPS, 4),
            "in_layer_how": gi["how"],
            "counters": "profiles/gemm_prefill_llama32_3b.md (rocprofv3 MfmaUtil per GEMM kind; shader clock of the "
                        "gate/up launches back to back and inside the layer)"}
    if not args.no_configs:
        del g16
        if "int8" in out:
            del g8
        log("other configs ...")
        res["configs"] = {
            "C1_tinyllama": decode_config_bench(torch, hi, "TinyLlama-1.1B decode GEMV set (22 distinct layers)",
                                                (2048, 32, 4, 64, 5632, 32000), [1], 22, args.steps, SEED + 10),
            "C4_qwen25_1p5b": decode_config_bench(torch, hi, "Qwen2.5-1.5B decode/verify GEMV set with QKV bias "
                                                  "(28 distinct layers), N rows", C4_DIMS,
                                                  [1, 2, 5, 8], 28, args.steps, SEED + 11, bias=True),
            "C5_granite_moe": moe_bench(torch, hi, args.steps, SEED + 12),
        }
    res["copy_bandwidth"] = copy_bandwidth(torch)
    if not args.no_cpu:
        log("cpu baseline ...")
        res["cpu_baseline"] = cpu_baseline(torch, model)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
