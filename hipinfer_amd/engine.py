"""Prefill and greedy decode of a dense Llama-family model over weights already in device memory,
built only from this library's C-ABI calls.

Follows the reference engine (src/api.cu): prefill (1807-1845) and decode_step (1891-1952), one
sequence per cache slot.

Prefill of T prompt tokens into slot s at positions p0.. (chunks of at most max_prefill rows):

    x = embed[tokens]                                     (embed_kernel, api.cu:1817)
    per layer l (attn_rows / mlp_rows, api.cu:1668-1713):
      qkv = RMSNorm(x; n1) @ Wqkv^T + bqkv                (hi_rmsnorm, hi_gemm epi 0)
      q rotated, K/V[s, p0..] = RoPE(k), v                (hi_rope_cache, prefill form)
      att = causal softmax(q K^T / sqrt(D)) V             (hi_flash_prefill over slot s)
      x  += att @ Wo^T                                    (hi_gemm epi 1)
      x  += SwiGLU(RMSNorm(x; n2) @ Wgu^T) @ Wdown^T      (hi_rmsnorm, hi_gemm epi 2, hi_gemm epi 1)
    logits[s] = RMSNorm(x[T-1]; nf) @ Wlm^T               (GEMV, api.cu:1829-1836)
    tok[s] = argmax(logits[s]); pos[s] = p0 + T

Decode step for slots 0..B-1 (tok and pos live on the device and advance there, so one captured
hipGraph replays step after step). Up to 8 sequences take the GEMV path with RMSNorm fused into
the projections; 9 to 64 the GEMM path (api.cu:1914-1940), whose tiles are tuned by the first,
eager step. From 2 sequences on, the first step also times the gate/up, down and lm_head
projections both ways and keeps, for each, the faster (the GEMM with a separate RMSNorm), as the
library's engine does:

    x = embed[tok]
    per layer l:
      GEMV: q, K/V[pos] = RoPE(RMSNorm(x; n1) @ Wqkv^T + bqkv)   (gemv_qkv_rope)
      GEMM: qkv = RMSNorm(x; n1) @ Wqkv^T + bqkv; RoPE + cache   (hi_rmsnorm, hi_gemm, hi_rope_cache)
      att = softmax(q K[0..pos]^T / sqrt(D)) V                    (hi_decode_attn)
      x  += att @ Wo^T
      x  += SwiGLU(RMSNorm(x; n2) @ Wgu^T) @ Wdown^T
    logits = RMSNorm(x; nf) @ Wlm^T
    tok = argmax(logits); pos += 1                                (greedy, kernels.cuh:1913-1931)

This class takes weights already in device memory (tests and benchmarks build them from seeds).
The weight-file path is the library's own engine (csrc/engine_api.hip: hi_load, hi_prefill,
hi_decode, hi_verify), which runs the same kernels in the same order and which hipinfer.Engine
wraps.
"""
import os

import torch

from . import hipinfer as hi

GEMV_MAX = 8  # sequences per decode step on the GEMV path (the library's HIPINFER_GEMV_MAX default)
GEMM_MAX = 64  # and on the batched-decode GEMM path
GU_GEMM, DOWN_GEMM, LM_GEMM = 1, 2, 4  # projections of a GEMV-path step that run on the GEMM


class DecodeStep:
    """cfg: dict with hidden H, heads Hq, kv heads Hkv, head_dim D, inter I, vocab V, layers L,
    eps, rope theta. weights: {"embed": [V, H], "lm": [V, H] or (int8, scales), "nf": [H],
    "layers": [{"qkv", "o", "gate_up", "down": [N, K] fp16 or (int8, scales); "bqkv": bias or None;
    "n1", "n2": [H]}]} with gate/up rows interleaved in groups of 16 (export.py:97-101).
    B: cache slots = sequences per decode step (1..64); max_prefill: rows per prefill chunk (0: no
    prefill buffers); small_gemm: for 2..8 sequences, the mask of projections (GU_GEMM, DOWN_GEMM,
    LM_GEMM) to run on the GEMM path, or None for the library engine's shape rule
    (small_paths_rule); the HIPINFER_SMALL_GEMM environment variable, when set, gives the mask
    instead, or with the value "tune" times both paths on the first eager step."""

    def __init__(self, cfg, weights, B, max_seq, max_prefill=0, small_gemm=None):
        assert 1 <= B <= GEMM_MAX, f"1..{GEMM_MAX} sequences per decode step"
        self.c, self.w, self.B, self.max_seq = dict(cfg), weights, B, max_seq
        self.gemm_path = B > GEMV_MAX
        env = os.environ.get("HIPINFER_SMALL_GEMM")
        if small_gemm is None and env and env != "tune":
            small_gemm = int(env) & 7
        if small_gemm is None and env != "tune":
            small_gemm = self.small_paths_rule(cfg, weights, B)
        self.small_gemm = 0 if (B == 1 or self.gemm_path) else small_gemm  # None: not timed yet
        H, Hq, Hkv, D, I, V, L = (cfg[k] for k in ("H", "Hq", "Hkv", "D", "I", "V", "L"))
        self.qkv_dim = (Hq + 2 * Hkv) * D
        dev = "cuda"
        f16 = torch.float16
        self.x = torch.zeros(B, H, dtype=f16, device=dev)
        self.q = torch.zeros(B, Hq * D, dtype=f16, device=dev)
        self.att = torch.zeros(B, Hq * D, dtype=f16, device=dev)
        self.act = torch.zeros(B, I, dtype=f16, device=dev)
        self.logits = torch.zeros(B, V, dtype=f16, device=dev)
        self.xn = torch.zeros(B, H, dtype=f16, device=dev)
        if self.gemm_path:
            self.qkv = torch.zeros(B, self.qkv_dim, dtype=f16, device=dev)
        self.kc = [torch.zeros(B, Hkv, max_seq, D, dtype=f16, device=dev) for _ in range(L)]
        self.vc = [torch.zeros_like(k) for k in self.kc]
        self.tok = torch.zeros(B, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(B, dtype=torch.int32, device=dev)
        self.work = torch.zeros(hi.lib.hi_decode_work_bytes(B, Hq, Hkv, D), dtype=torch.uint8, device=dev)
        theta = float(cfg.get("theta", 10000.0))
        inv = 1.0 / theta ** (torch.arange(0, D, 2, device=dev, dtype=torch.float64) / D)
        ang = torch.arange(max_seq, device=dev, dtype=torch.float64)[:, None] * inv[None, :]
        self.cs = torch.stack([ang.cos(), ang.sin()], -1).to(f16).contiguous()  # [max_seq, D/2, 2]
        self.max_prefill = max_prefill
        if max_prefill:
            P = max_prefill
            self.px = torch.zeros(P, H, dtype=f16, device=dev)
            self.pxn = torch.zeros(P, H, dtype=f16, device=dev)
            self.pqkv = torch.zeros(P, self.qkv_dim, dtype=f16, device=dev)
            self.patt = torch.zeros(P, Hq * D, dtype=f16, device=dev)
            self.pact = torch.zeros(P, I, dtype=f16, device=dev)
            self.ptok = torch.zeros(P, dtype=torch.int32, device=dev)

    @staticmethod
    def _ws(W):
        return (W[0], W[1]) if isinstance(W, tuple) else (W, None)

    def _attn_mlp_gemm(self, ly, att, x, xn, act, eps, next_norm):
        """x += o(att); x += SwiGLU(RMSNorm(x; n2) @ Wgu^T) @ Wdown^T on the GEMM (rows of x), each
        residual GEMM with the RMSNorm that reads its result (n2 after o; next_norm, the next layer's
        n1 or the final norm, after down) in one call. Leaves RMSNorm(x; next_norm) in xn."""
        Wo, so = self._ws(ly["o"])
        hi.gemm_rmsnorm(att, Wo, x, ly["n2"], eps, out=xn, scales=so)
        Wg, sg = self._ws(ly["gate_up"])
        hi.gemm(xn, Wg, out=act, epi=2, scales=sg)
        Wd, sd = self._ws(ly["down"])
        hi.gemm_rmsnorm(act, Wd, x, next_norm, eps, out=xn, scales=sd)

    @staticmethod
    def small_paths_rule(cfg, weights, B):
        """The projections of a B-sequence GEMV-path step that run on the GEMM, by the library
        engine's fixed shape rule (engine_api.hip small_paths_rule): down when its B activation rows
        do not fit one GEMV launch's LDS (the launch would run in row chunks) or, with int8 weights,
        from 5 rows on; lm_head with int8 weights at 8 rows. gate/up, QKV and o stay on the
        GEMV."""
        if B < 2:
            return 0
        mask = 0
        dq8 = isinstance(weights["layers"][0]["down"], tuple)
        fit = hi.lib.hi_gemv_rows_per_launch(cfg["I"], 0, int(dq8))
        if fit < 0:
            raise RuntimeError(f"hi_gemv_rows_per_launch failed ({fit})")
        if B > fit or (dq8 and B >= 5):
            mask |= DOWN_GEMM
        if isinstance(weights["lm"], tuple) and B >= 8:
            mask |= LM_GEMM
        return mask

    def _tune_small_paths(self, eps):
        """Time gate/up, down and lm_head on the GEMV path and on the GEMM path (with the RMSNorm
        the GEMV fuses), on scratch rows and the weights of up to 8 layers in turn; keep the GEMM
        where it is at least 3 % faster."""
        w, B = self.w, self.B
        lys = w["layers"][:8]
        reps = max(8, 2 * len(lys))
        xs, x2 = torch.zeros_like(self.x), torch.zeros_like(self.x)
        xn, act, lg = torch.zeros_like(self.xn), torch.zeros_like(self.act), torch.zeros_like(self.logits)

        def time_us(fn, n):
            for i in range(min(n, 2)):  # untimed: also tunes the GEMM tiles of these shapes
                fn(i)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for r in range(reps):
                fn(r % n)
            e1.record()
            e1.synchronize()
            return e0.elapsed_time(e1) * 1e3 / reps

        def pick(bit, gemv_fn, gemm_fn, n):
            return bit if time_us(gemm_fn, n) < 0.97 * time_us(gemv_fn, n) else 0

        def gu_gemm(i):
            hi.rmsnorm(xs, lys[i]["n2"], eps, out=xn)
            Wg, sg = self._ws(lys[i]["gate_up"])
            hi.gemm(xn, Wg, out=act, epi=2, scales=sg)

        def lm_gemm(i):
            hi.rmsnorm(xs, w["nf"], eps, out=xn)
            hi.gemm(xn, Wl, out=lg, scales=sl)

        Wl, sl = self._ws(w["lm"])
        mask = pick(GU_GEMM, lambda i: hi.gemv(xs, self._ws(lys[i]["gate_up"])[0], out=act, normw=lys[i]["n2"],
                                               eps=eps, epi=2, scales=self._ws(lys[i]["gate_up"])[1]),
                    gu_gemm, len(lys))
        mask |= pick(DOWN_GEMM, lambda i: hi.gemv(act, self._ws(lys[i]["down"])[0], out=x2, epi=1,
                                                  scales=self._ws(lys[i]["down"])[1]),
                     lambda i: hi.gemm(act, self._ws(lys[i]["down"])[0], out=x2, epi=1,
                                       scales=self._ws(lys[i]["down"])[1]), len(lys))
        mask |= pick(LM_GEMM, lambda i: hi.gemv(xs, Wl, out=lg, normw=w["nf"], eps=eps, scales=sl), lm_gemm, 1)
        return mask

    def step(self):
        """One token for every slot: reads tok / pos, writes the next tok, advances pos."""
        c, w = self.c, self.w
        eps = float(c.get("eps", 1e-5))
        Hq, Hkv, D = c["Hq"], c["Hkv"], c["D"]
        if self.small_gemm is None:  # a capture before the first eager step keeps the GEMVs
            self.small_gemm = 0 if torch.cuda.is_current_stream_capturing() else self._tune_small_paths(eps)
        sg = self.small_gemm
        hi.embed(self.tok, w["embed"], out=self.x)
        layers = w["layers"]
        if self.gemm_path:  # later layers' norm (and the final one) come with the previous down GEMM
            hi.rmsnorm(self.x, layers[0]["n1"], eps, out=self.xn)
        for l, ly in enumerate(layers):
            Wq, sq = self._ws(ly["qkv"])
            if self.gemm_path:
                hi.gemm(self.xn, Wq, out=self.qkv, bias=ly.get("bqkv"), scales=sq)
                hi.rope_cache(self.qkv, Hq, Hkv, self.cs, self.kc[l], self.vc[l], pos=self.pos)
                q = self.qkv[:, :Hq * D]
            else:
                hi.gemv_qkv_rope(self.x, Wq, ly["n1"], Hq, Hkv, self.cs, self.pos, self.kc[l], self.vc[l], self.q,
                                 bias=ly.get("bqkv"), eps=eps, scales=sq)
                q = self.q
            hi.decode_attn(q, self.kc[l], self.vc[l], self.pos, Hq, Hkv, out=self.att, work=self.work)
            if self.gemm_path:
                nxt = layers[l + 1]["n1"] if l + 1 < len(layers) else w["nf"]
                self._attn_mlp_gemm(ly, self.att, self.x, self.xn, self.act, eps, nxt)
            else:
                Wo, so = self._ws(ly["o"])
                hi.gemv(self.att, Wo, out=self.x, epi=1, scales=so)
                Wg, s_g = self._ws(ly["gate_up"])
                if sg & GU_GEMM:
                    hi.rmsnorm(self.x, ly["n2"], eps, out=self.xn)
                    hi.gemm(self.xn, Wg, out=self.act, epi=2, scales=s_g)
                else:
                    hi.gemv(self.x, Wg, out=self.act, normw=ly["n2"], eps=eps, epi=2, scales=s_g)
                Wd, sd = self._ws(ly["down"])
                if sg & DOWN_GEMM:
                    hi.gemm(self.act, Wd, out=self.x, epi=1, scales=sd)
                else:
                    hi.gemv(self.act, Wd, out=self.x, epi=1, scales=sd)
        Wl, sl = self._ws(w["lm"])
        if self.gemm_path or sg & LM_GEMM:
            if not self.gemm_path:
                hi.rmsnorm(self.x, w["nf"], eps, out=self.xn)
            hi.gemm(self.xn, Wl, out=self.logits, scales=sl)
        else:
            hi.gemv(self.x, Wl, out=self.logits, normw=w["nf"], eps=eps, scales=sl)
        hi.argmax(self.logits, out=self.tok)
        self.pos.add_(1)

    def capture(self):
        """The step as a hipGraph (replay it to decode; tok / pos advance on the device). Run one
        eager step first: neither the GEMM tile tuning nor the timing of the 2-8-sequence paths runs
        under capture (a capture before it keeps those projections on the GEMV)."""
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step()
        return g

    def prefill(self, slot, tokens, p0=0):
        """Prefill the prompt `tokens` (host ints) into cache slot `slot` at positions p0..; leaves the
        last position's logits in logits[slot], the greedy next token in tok[slot] and its position
        p0 + len(tokens) in pos[slot]. Returns that token."""
        c, w = self.c, self.w
        T = len(tokens)
        assert self.max_prefill > 0, "built without prefill buffers (max_prefill=0)"
        assert 0 <= slot < self.B and T >= 1 and 0 <= p0 and p0 + T <= self.max_seq
        eps = float(c.get("eps", 1e-5))
        Hq, Hkv, D = c["Hq"], c["Hkv"], c["D"]
        toks = torch.as_tensor(list(tokens), dtype=torch.int32)
        for t0 in range(0, T, self.max_prefill):
            n = min(self.max_prefill, T - t0)
            pb = p0 + t0
            self.ptok[:n].copy_(toks[t0:t0 + n])
            x, xn, qkv, att, act = self.px[:n], self.pxn[:n], self.pqkv[:n], self.patt[:n], self.pact[:n]
            hi.embed(self.ptok[:n], w["embed"], out=x)
            layers = w["layers"]
            hi.rmsnorm(x, layers[0]["n1"], eps, out=xn)  # later layers': the previous down GEMM's call
            for l, ly in enumerate(layers):
                Wq, sq = self._ws(ly["qkv"])
                hi.gemm(xn, Wq, out=qkv, bias=ly.get("bqkv"), scales=sq)
                hi.rope_cache(qkv, Hq, Hkv, self.cs, self.kc[l], self.vc[l], pos_base=pb, slot_base=slot)
                hi.flash_prefill(qkv[:, :Hq * D], self.kc[l][slot], self.vc[l][slot], n, pb, Hq, Hkv, out=att)
                nxt = layers[l + 1]["n1"] if l + 1 < len(layers) else w["nf"]
                self._attn_mlp_gemm(ly, att, x, xn, act, eps, nxt)
        Wl, sl = self._ws(w["lm"])
        hi.gemv(x[n - 1:n], Wl, out=self.logits[slot:slot + 1], normw=w["nf"], eps=eps, scales=sl)
        hi.argmax(self.logits[slot:slot + 1], out=self.tok[slot:slot + 1])
        self.pos[slot:slot + 1].fill_(p0 + T)
        return int(self.tok[slot].item())
