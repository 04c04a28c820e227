"""Greedy decode step of a dense Llama-family model over weights already in device memory, built
only from this library's C-ABI calls.

Follows the reference engine's decode_step (src/api.cu:1891-1952) on its GEMV path (batch up to 8,
RMSNorm fused into the projections), one sequence per cache slot:

    x = embed[tok]                                        (embed_kernel, api.cu:1900)
    per layer l:
      q, K/V[pos] = RoPE(RMSNorm(x; n1) @ Wqkv^T + bqkv)  (gemv_qkv_rope, 1907-1914)
      att = softmax(q K[0..pos]^T / sqrt(D)) V            (hi_decode_attn, 1921)
      x  += att @ Wo^T                                    (gemv epi 1, 1929)
      act = SwiGLU(RMSNorm(x; n2) @ Wgu^T)                (gemv epi 2, 1931)
      x  += act @ Wdown^T                                 (gemv epi 1, 1933)
    logits = RMSNorm(x; nf) @ Wlm^T                       (1942)
    tok = argmax(logits); pos += 1                        (greedy / emit_token, 1948, kernels.cuh:1913-1931)

tok and pos live on the device and advance there, so one captured hipGraph replays step after step.
The weight-file loader and the prefill that the reference's hi_load / hi_prefill add around this
step are not part of this package; a caller supplies the weights and fills the caches.
"""
import torch

from . import hipinfer as hi


class DecodeStep:
    """cfg: dict with hidden H, heads Hq, kv heads Hkv, head_dim D, inter I, vocab V, layers L,
    eps, rope theta. weights: {"embed": [V, H], "lm": [V, H] or (int8, scales), "nf": [H],
    "layers": [{"qkv", "o", "gate_up", "down": [N, K] fp16 or (int8, scales); "bqkv": bias or None;
    "n1", "n2": [H]}]} with gate/up rows interleaved in groups of 16 (export.py:97-101)."""

    def __init__(self, cfg, weights, B, max_seq):
        assert 1 <= B <= 8, "the GEMV path serves up to 8 sequences"
        self.c, self.w, self.B, self.max_seq = dict(cfg), weights, B, max_seq
        H, Hq, Hkv, D, I, V, L = (cfg[k] for k in ("H", "Hq", "Hkv", "D", "I", "V", "L"))
        dev = "cuda"
        f16 = torch.float16
        self.x = torch.zeros(B, H, dtype=f16, device=dev)
        self.q = torch.zeros(B, Hq * D, dtype=f16, device=dev)
        self.att = torch.zeros(B, Hq * D, dtype=f16, device=dev)
        self.act = torch.zeros(B, I, dtype=f16, device=dev)
        self.logits = torch.zeros(B, V, dtype=f16, device=dev)
        self.kc = [torch.zeros(B, Hkv, max_seq, D, dtype=f16, device=dev) for _ in range(L)]
        self.vc = [torch.zeros_like(k) for k in self.kc]
        self.tok = torch.zeros(B, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(B, dtype=torch.int32, device=dev)
        self.work = torch.zeros(hi.lib.hi_decode_work_bytes(B, Hq, Hkv, D), dtype=torch.uint8, device=dev)
        theta = float(cfg.get("theta", 10000.0))
        inv = 1.0 / theta ** (torch.arange(0, D, 2, device=dev, dtype=torch.float64) / D)
        ang = torch.arange(max_seq, device=dev, dtype=torch.float64)[:, None] * inv[None, :]
        self.cs = torch.stack([ang.cos(), ang.sin()], -1).to(f16).contiguous()  # [max_seq, D/2, 2]

    @staticmethod
    def _ws(W):
        return (W[0], W[1]) if isinstance(W, tuple) else (W, None)

    def step(self):
        """One token for every slot: reads tok / pos, writes the next tok, advances pos."""
        c, w = self.c, self.w
        eps = float(c.get("eps", 1e-5))
        hi.embed(self.tok, w["embed"], out=self.x)
        for l, ly in enumerate(w["layers"]):
            Wq, sq = self._ws(ly["qkv"])
            hi.gemv_qkv_rope(self.x, Wq, ly["n1"], c["Hq"], c["Hkv"], self.cs, self.pos, self.kc[l], self.vc[l], self.q,
                             bias=ly.get("bqkv"), eps=eps, scales=sq)
            hi.decode_attn(self.q, self.kc[l], self.vc[l], self.pos, c["Hq"], c["Hkv"], out=self.att, work=self.work)
            Wo, so = self._ws(ly["o"])
            hi.gemv(self.att, Wo, out=self.x, epi=1, scales=so)
            Wg, sg = self._ws(ly["gate_up"])
            hi.gemv(self.x, Wg, out=self.act, normw=ly["n2"], eps=eps, epi=2, scales=sg)
            Wd, sd = self._ws(ly["down"])
            hi.gemv(self.act, Wd, out=self.x, epi=1, scales=sd)
        Wl, sl = self._ws(w["lm"])
        hi.gemv(self.x, Wl, out=self.logits, normw=w["nf"], eps=eps, scales=sl)
        hi.argmax(self.logits, out=self.tok)
        self.pos.add_(1)

    def capture(self):
        """The step as a hipGraph (replay it to decode; tok / pos advance on the device)."""
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step()
        return g
