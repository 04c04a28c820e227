"""Python face of libhipinfer.so: the hipinfer matmul hot path (and the engine built on it) called
on torch tensors that live on an MI355X.

The public names, argument order, defaults and return values are those of the reference's
Python module (scripts/hipinfer.py: rmsnorm, gemv, gemv_qkv_rope, gemm, moe_router, moe_experts,
decode_attn, rope_cache, flash_prefill, flash_prefill_lse, Engine), so code written against it
runs here unchanged; the int8 weight tools of scripts/export.py:54-101 (quantize_rows,
dequantize_rows, interleave_gate_up) are here too, the first two running on the GPU.

How this module is put together:
  * the C-ABI is declared once, below, as C prototypes (the same text as include/hipinfer.h);
    a small parser turns each prototype into ctypes argtypes / restype, and a CPU test checks the
    table against the header, so the two cannot drift apart;
  * every wrapper validates its tensors (device, dtype, rank, row layout) before any launch, then
    makes one C call on torch's current stream; a non-zero code from the library (it prints the
    reason on stderr) becomes ValueError;
  * torch only provides device memory and the stream: there is no CPU path. Importing fails when
    the library is not built, and every call needs the GPU.
"""
import ctypes
import os
import re

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.abspath(os.environ.get("HIPINFER_LIB", os.path.join(_HERE, "libhipinfer.so")))
if not os.path.exists(LIBRARY_PATH):
    raise ImportError(f"hipinfer_amd: {LIBRARY_PATH} is not built; run `python -m hipinfer_amd.build`")
# torch ships its own HIP runtime and this library links the system one; the two share the process
# only when torch's is initialised first, so make sure it is before the library is loaded
torch.cuda.is_available()
lib = ctypes.CDLL(LIBRARY_PATH)

# moe_flags bits (the reference's MOE_NORM_TOPK / MOE_FP16_WEIGHTS): softmax over the chosen k
# instead of all experts; routing weights rounded to fp16.
MOE_NORM_TOPK = 1
MOE_FP16_WEIGHTS = 2

# ------------------------------------------------------------------ the C-ABI, as prototypes
ABI = """
int hi_rmsnorm(ptr x, ptr w, ptr y, int M, int H, float eps, ptr stream);
int hi_gemv(ptr x, int ldx, ptr normw, float eps, ptr W, ptr out, int ldo, int M, int N, int K, int epi, ptr stream);
int hi_gemv_w8(ptr x, int ldx, ptr normw, float eps, ptr W, ptr scales, ptr out, int ldo, int M, int N, int K,
               int epi, ptr stream);
int hi_gemv_qkv_rope(ptr x, int ldx, ptr normw, float eps, ptr W, ptr bias, ptr out, int ldo, int M, int K, int Hq,
                     int Hkv, int D, ptr cs, ptr pos, ptr kc, ptr vc, int max_seq, ptr stream);
int hi_gemv_qkv_rope_w8(ptr x, int ldx, ptr normw, float eps, ptr W, ptr scales, ptr bias, ptr out, int ldo, int M,
                        int K, int Hq, int Hkv, int D, ptr cs, ptr pos, ptr kc, ptr vc, int max_seq, ptr stream);
int hi_quantize_rows(ptr w, i64 N, int K, ptr q, ptr s, ptr stream);
int hi_dequantize_rows(ptr q, ptr s, i64 N, int K, ptr out, ptr stream);
int hi_device_cus();
int hi_max_smem();
int hi_gemv_rows_per_launch(int K, int norm, int int8);
int hi_gemm(ptr A, int lda, ptr W, ptr bias, ptr C, int ldc, int M, int N, int K, int epi, ptr stream);
int hi_gemm_w8(ptr A, int lda, ptr W, ptr scales, ptr bias, ptr C, int ldc, int M, int N, int K, int epi, ptr stream);
int hi_gemm_force_config(int cfg);
int hi_gemm_force_splits(int splits);
int hi_gemm_num_configs();
int hi_gemm_config_desc(int cfg, str out, int n);
int hi_gemm_last_choice(ptr cfg, ptr splits);
int hi_gemm_residual_rmsnorm(ptr A, int lda, ptr W, ptr scales, ptr X, int M, int N, int K, ptr norm_w, float eps,
                             ptr Y, ptr stream);
int hi_gemm_noalloc(ptr A, int lda, ptr W, ptr scales, ptr bias, ptr C, int ldc, int M, int N, int K, int epi,
                    ptr stream);
int hi_moe_router(ptr xn, int ldx, ptr Wr, int M, int E, int H, int k, int flags, ptr idx, ptr w, ptr stream);
size hi_moe_work_bytes(int M, int k, int E, int H, int I);
int hi_moe_experts(ptr xn, int ldxn, ptr wgu, ptr wdown, ptr idx, ptr w, int M, int E, int k, int H, int I, int flags,
                   float scale, ptr x, int ldx, int path, ptr work, ptr stream);
int hi_moe_route_experts(ptr xn, int ldxn, ptr Wr, ptr wgu, ptr wdown, int M, int E, int k, int H, int I, int flags,
                         float scale, ptr x, int ldx, ptr idx, ptr w, ptr work, ptr stream);
size hi_decode_work_bytes(int B, int Hq, int Hkv, int D);
int hi_decode_attn(ptr q, int ldq, ptr kc, ptr vc, int max_seq, ptr pos, ptr out, int ldo, int B, int Hq, int Hkv,
                   int D, ptr work, ptr stream);
int hi_argmax(ptr logits, int B, int V, ptr tok, ptr stream);
int hi_embed(ptr tok, ptr table, int V, int H, ptr x, int ldx, int B, ptr stream);
int hi_rope_cache(ptr qkv, int ldq, int M, int Hq, int Hkv, int D, ptr cs, ptr pos, int pos_base, int slot_base,
                  ptr kc, ptr vc, int max_seq, ptr stream);
int hi_flash_prefill(ptr q, int ldq, ptr kc, ptr vc, int max_seq, ptr out, int ldo, int T, int p0, int Hq, int Hkv,
                     int D, ptr stream);
int hi_flash_prefill_lse(ptr q, int ldq, ptr kc, ptr vc, int max_seq, ptr out, int ldo, int T, int p0, int Hq,
                         int Hkv, int D, ptr lse, ptr stream);
ptr hi_load(str path, int max_batch, int max_seq, int max_prefill);
ptr hi_load_tp(str path, int max_batch, int max_seq, int max_prefill, int world, ptr devs);
void hi_free(ptr e);
void hi_config(ptr e, ptr out);
void hi_moe_config(ptr e, ptr out);
size hi_weight_bytes(ptr e);
int hi_weight_quant(ptr e);
int hi_prefill(ptr e, int slot, ptr tokens, int T, int p0);
int hi_prefill_logits(ptr e, int slot, ptr tokens, int T, int p0, ptr logits);
float hi_decode(ptr e, int B, int steps, int use_graph);
int hi_history(ptr e, int slot, int start, int n, ptr out);
int hi_logits(ptr e, int B, ptr out);
int hi_set_state(ptr e, int B, ptr tokens, ptr positions);
int hi_rewind(ptr e, int slot, int len, int tok);
void hi_sync(ptr e);
ptr hi_stream(ptr e);
int hi_verify_max_rows();
int hi_verify(ptr e, int slot, ptr tokens, int R, int p0, ptr out, ptr logits, int use_graph);
"""

_CTYPE = {"int": ctypes.c_int, "i64": ctypes.c_longlong, "float": ctypes.c_float, "size": ctypes.c_size_t,
          "ptr": ctypes.c_void_p, "str": ctypes.c_char_p, "void": None}


def parse_abi(text):
    """{name: (return kind, [argument kinds])} from prototypes `kind name(kind arg, ...);`."""
    decls = {}
    for m in re.finditer(r"(\w+)\s+(hi_\w+)\s*\(([^)]*)\)\s*;", text):
        args = [a.split()[0] for a in m.group(3).split(",") if a.strip()]
        decls[m.group(2)] = (m.group(1), args)
    return decls


SIGNATURES = parse_abi(ABI)
for _name, (_ret, _args) in SIGNATURES.items():
    _fn = getattr(lib, _name)  # every prototype must exist in the library
    _fn.restype = _CTYPE[_ret]
    _fn.argtypes = [_CTYPE[a] for a in _args]


# ------------------------------------------------------------------ call helpers
def ptr(t):
    """Device address of a tensor (None passes NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def cur_stream():
    """torch's current HIP stream, as the library's `stream` argument."""
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def check_rc(rc, what):
    """A library return code: 0 is success; the library printed the reason for anything else."""
    if rc != 0:
        raise ValueError(f"hipinfer_amd.{what}: the library rejected the call (code {rc}; reason on stderr)")
    return rc


def _need(what, t, dtype=None, ndim=None, rows=False, optional=False):
    """Checks one tensor argument: on a GPU, of the given dtype and rank; rows=True also needs unit
    stride along the last dimension (rows may be strided, as leading dimensions allow)."""
    if t is None:
        if optional:
            return
        raise ValueError(f"hipinfer_amd.{what}: a tensor argument is missing")
    if not t.is_cuda:
        raise ValueError(f"hipinfer_amd.{what}: tensors must live on the GPU (got {t.device})")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"hipinfer_amd.{what}: expected {dtype}, got {t.dtype}")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"hipinfer_amd.{what}: expected {ndim} dimensions, got shape {tuple(t.shape)}")
    if rows and t.stride(-1) != 1:
        raise ValueError(f"hipinfer_amd.{what}: rows must be contiguous")


def _weight(what, W, scales):
    """A [N, K] projection: fp16, or int8 with one fp16 scale per row. Returns True for int8."""
    _need(what, W, ndim=2, rows=True)
    if scales is None:
        if W.dtype != torch.float16:
            raise ValueError(f"hipinfer_amd.{what}: fp16 weights, or int8 weights with scales")
        return False
    _need(what, scales, torch.float16, 1)
    if W.dtype != torch.int8 or scales.shape[0] != W.shape[0]:
        raise ValueError(f"hipinfer_amd.{what}: int8 weights need one fp16 scale per row")
    return True


def _alloc_rows(ref, M, N, dtype=torch.float16):
    return torch.empty(M, N, dtype=dtype, device=ref.device)


# ------------------------------------------------------------------ kernels
def rmsnorm(x, w, eps=1e-5, out=None):
    """RMSNorm of each row of x [M, H]: w * fp16(x * rsqrt(mean(x^2) + eps)), HF rounding order."""
    y = torch.empty_like(x) if out is None else out
    for t in (x, w, y):
        _need("rmsnorm", t, torch.float16)
    if not (x.is_contiguous() and y.is_contiguous()):
        raise ValueError("hipinfer_amd.rmsnorm: rows of x and out must be packed")
    check_rc(lib.hi_rmsnorm(ptr(x), ptr(w), ptr(y), x.shape[0], x.shape[1], eps, cur_stream()), "rmsnorm")
    return y


def gemv(x, W, out=None, normw=None, eps=1e-5, epi=0, scales=None):
    """Decode GEMV for a few activation rows x [M, K] against W [N, K]:
    epi 0 writes x W^T, epi 1 adds it to out (residual), epi 2 writes the SwiGLU of gate/up row pairs
    (W's rows interleaved in groups of 16; out is N/2 wide). normw fuses an RMSNorm of x first."""
    _need("gemv", x, torch.float16, 2, rows=True)
    q8 = _weight("gemv", W, scales)
    _need("gemv", normw, torch.float16, 1, optional=True)
    M, K = x.shape
    N = W.shape[0]
    if out is None:
        out = _alloc_rows(x, M, N // 2 if epi == 2 else N)
    _need("gemv", out, torch.float16, 2, rows=True)
    head = (ptr(x), x.stride(0), ptr(normw), eps, ptr(W))
    tail = (ptr(out), out.stride(0), M, N, K, epi, cur_stream())
    rc = lib.hi_gemv_w8(*head, ptr(scales), *tail) if q8 else lib.hi_gemv(*head, *tail)
    check_rc(rc, "gemv")
    return out


def gemv_qkv_rope(x, W, normw, Hq, Hkv, cs, pos, kc, vc, out, bias=None, eps=1e-5, scales=None):
    """The decode QKV projection with everything after it fused: RMSNorm(x) @ W^T (+ bias), RoPE on q
    and k, q into out [M, Hq*D], k / v of row m into cache slot m at position pos[m]
    (kc, vc: [slots, Hkv, max_seq, D]; cs: [max_seq, D/2, 2] cos/sin)."""
    _need("gemv_qkv_rope", x, torch.float16, 2, rows=True)
    q8 = _weight("gemv_qkv_rope", W, scales)
    for t in (kc, vc):
        _need("gemv_qkv_rope", t, torch.float16, 4)
    _need("gemv_qkv_rope", pos, torch.int32, 1)
    _need("gemv_qkv_rope", out, torch.float16, 2, rows=True)
    _need("gemv_qkv_rope", bias, torch.float16, 1, optional=True)
    M, K = x.shape
    D, max_seq = kc.shape[3], kc.shape[2]
    head = (ptr(x), x.stride(0), ptr(normw), eps, ptr(W))
    tail = (ptr(bias), ptr(out), out.stride(0), M, K, Hq, Hkv, D, ptr(cs), ptr(pos), ptr(kc), ptr(vc), max_seq,
            cur_stream())
    rc = lib.hi_gemv_qkv_rope_w8(*head, ptr(scales), *tail) if q8 else lib.hi_gemv_qkv_rope(*head, *tail)
    check_rc(rc, "gemv_qkv_rope")
    return out


def gemm(A, W, out=None, epi=0, bias=None, scales=None):
    """Prefill GEMM on the matrix cores: A [M, K] @ W^T with epilogue epi (0 store, + bias when given;
    1 add into out; 2 SwiGLU over interleaved gate/up rows, out N/2 wide)."""
    _need("gemm", A, torch.float16, 2, rows=True)
    q8 = _weight("gemm", W, scales)
    _need("gemm", bias, torch.float16, 1, optional=True)
    M, K = A.shape
    N = W.shape[0]
    if out is None:
        out = _alloc_rows(A, M, N // 2 if epi == 2 else N)
    _need("gemm", out, torch.float16, 2, rows=True)
    head = (ptr(A), A.stride(0), ptr(W))
    tail = (ptr(bias), ptr(out), out.stride(0), M, N, K, epi, cur_stream())
    rc = lib.hi_gemm_w8(*head, ptr(scales), *tail) if q8 else lib.hi_gemm(*head, *tail)
    check_rc(rc, "gemm")
    return out


def gemm_rmsnorm(A, W, x, normw, eps=1e-5, out=None, scales=None):
    """x += A @ W^T (the residual epilogue), then RMSNorm of the new x into out: the same bits as
    gemm(A, W, out=x, epi=1) followed by rmsnorm(x, normw), with the norm inside the split-K second
    pass when the GEMM splits K. x and out packed [M, N]."""
    _need("gemm_rmsnorm", A, torch.float16, 2, rows=True)
    _weight("gemm_rmsnorm", W, scales)
    for t in (x, normw):
        _need("gemm_rmsnorm", t, torch.float16)
    y = torch.empty_like(x) if out is None else out
    _need("gemm_rmsnorm", y, torch.float16)
    if not (x.is_contiguous() and y.is_contiguous()):
        raise ValueError("hipinfer_amd.gemm_rmsnorm: rows of x and out must be packed")
    M, K = A.shape
    check_rc(lib.hi_gemm_residual_rmsnorm(ptr(A), A.stride(0), ptr(W), ptr(scales), ptr(x), M, W.shape[0], K,
                                          ptr(normw), eps, ptr(y), cur_stream()), "gemm_rmsnorm")
    return y


def gemm_noalloc(A, W, out, epi=0, bias=None, scales=None):
    """gemm into a caller-provided `out` through the library's entry point that allocates no device
    memory (safe under graph capture and in allocation-free loops): split-K partials use the
    library's 64 MB static scratch, the tile comes from earlier tuning or the cost model. Calls that
    overlap in time on one GPU race on that scratch."""
    _need("gemm_noalloc", A, torch.float16, 2, rows=True)
    _weight("gemm_noalloc", W, scales)
    _need("gemm_noalloc", bias, torch.float16, 1, optional=True)
    _need("gemm_noalloc", out, torch.float16, 2, rows=True)
    M, K = A.shape
    check_rc(lib.hi_gemm_noalloc(ptr(A), A.stride(0), ptr(W), ptr(scales), ptr(bias), ptr(out), out.stride(0), M,
                                 W.shape[0], K, epi, cur_stream()), "gemm_noalloc")
    return out


def _routing(xn, M, k):
    return (torch.empty(M, k, dtype=torch.int32, device=xn.device),
            torch.empty(M, k, dtype=torch.float32, device=xn.device))


def _moe_work(xn, M, k, E, H, I, zeroed=False):
    """The expert work buffer; moe_route_experts needs it zeroed (its first 2304 bytes are arrival
    counters that must start consistent)."""
    make = torch.zeros if zeroed else torch.empty
    return make(lib.hi_moe_work_bytes(M, k, E, H, I), dtype=torch.uint8, device=xn.device)


def moe_router(xn, Wr, k, flags):
    """Routing of normalised rows xn [M, H] by router weights Wr [E, H]: the top k experts of each
    row, best first, as (idx [M, k] int32, weights [M, k] fp32)."""
    _need("moe_router", xn, torch.float16, 2, rows=True)
    _need("moe_router", Wr, torch.float16, 2, rows=True)
    M, H = xn.shape
    idx, w = _routing(xn, M, k)
    check_rc(lib.hi_moe_router(ptr(xn), xn.stride(0), ptr(Wr), M, Wr.shape[0], H, k, flags, ptr(idx), ptr(w),
                               cur_stream()), "moe_router")
    return idx, w


def moe_experts(xn, wgu, wdown, idx, w, x, flags, scale=1.0, path=0):
    """Adds the routed experts' SwiGLU MLPs to x in place: wgu [E, 2I, H] (gate/up interleaved by
    16 rows), wdown [E, H, I]; path 0 chooses, 1 forces the GEMV kernels, 2 the grouped GEMM."""
    for t in (xn, x):
        _need("moe_experts", t, torch.float16, 2, rows=True)
    for t in (wgu, wdown):
        _need("moe_experts", t, torch.float16, 3)
    M, H = xn.shape
    E, I, k = wgu.shape[0], wdown.shape[2], idx.shape[1]
    work = _moe_work(xn, M, k, E, H, I)
    check_rc(lib.hi_moe_experts(ptr(xn), xn.stride(0), ptr(wgu), ptr(wdown), ptr(idx), ptr(w), M, E, k, H, I, flags,
                                scale, ptr(x), x.stride(0), path, ptr(work), cur_stream()), "moe_experts")
    return x


def moe_route_experts(xn, Wr, wgu, wdown, k, x, flags, scale=1.0):
    """moe_router followed by moe_experts(path=0) as one library call with the same results: one row
    runs as a single launch when its grid fits on the GPU at once, else on the GEMV path (up to
    HIPINFER_GEMV_MAX rows) the routing runs inside the gate/up launch. Returns the routing
    (idx, weights)."""
    for t in (xn, x):
        _need("moe_route_experts", t, torch.float16, 2, rows=True)
    M, H = xn.shape
    E, I = wgu.shape[0], wdown.shape[2]
    idx, w = _routing(xn, M, k)
    work = _moe_work(xn, M, k, E, H, I, zeroed=True)
    check_rc(lib.hi_moe_route_experts(ptr(xn), xn.stride(0), ptr(Wr), ptr(wgu), ptr(wdown), M, E, k, H, I, flags,
                                      scale, ptr(x), x.stride(0), ptr(idx), ptr(w), ptr(work), cur_stream()),
             "moe_route_experts")
    return idx, w


def decode_attn(q, kc, vc, pos, Hq, Hkv, out=None, work=None):
    """One decode step of attention: sequence b's query q[b] [Hq*D] over the keys and values 0..pos[b]
    of cache slot b (kc, vc: [B, Hkv, max_seq, D]). `work` (zeroed once, hi_decode_work_bytes) can be
    reused across calls: the kernel leaves its counters at zero."""
    _need("decode_attn", q, torch.float16, 2, rows=True)
    for t in (kc, vc):
        _need("decode_attn", t, torch.float16, 4)
    _need("decode_attn", pos, torch.int32, 1)
    B, D, max_seq = q.shape[0], kc.shape[3], kc.shape[2]
    if out is None:
        out = _alloc_rows(q, B, Hq * D)
    if work is None:
        work = torch.zeros(lib.hi_decode_work_bytes(B, Hq, Hkv, D), dtype=torch.uint8, device=q.device)
    check_rc(lib.hi_decode_attn(ptr(q), q.stride(0), ptr(kc), ptr(vc), max_seq, ptr(pos), ptr(out), out.stride(0), B,
                                Hq, Hkv, D, ptr(work), cur_stream()), "decode_attn")
    return out


def rope_cache(qkv, Hq, Hkv, cs, kc, vc, pos=None, pos_base=0, slot_base=0):
    """After a QKV GEMM: rotates the q heads of qkv [M, (Hq+2Hkv)*D] in place and writes the rotated
    k and the v of row m to the cache. Decode form (pos given): slot slot_base + m, position pos[m];
    prefill form: slot slot_base, position pos_base + m."""
    _need("rope_cache", qkv, torch.float16, 2, rows=True)
    _need("rope_cache", pos, torch.int32, 1, optional=True)
    D, max_seq = kc.shape[3], kc.shape[2]
    check_rc(lib.hi_rope_cache(ptr(qkv), qkv.stride(0), qkv.shape[0], Hq, Hkv, D, ptr(cs), ptr(pos), pos_base,
                               slot_base, ptr(kc), ptr(vc), max_seq, cur_stream()), "rope_cache")


def _flash(q, kc, vc, T, p0, Hq, Hkv, out, lse):
    _need("flash_prefill", q, torch.float16, 2, rows=True)
    for t in (kc, vc):
        _need("flash_prefill", t, torch.float16, 3)
    D, max_seq = kc.shape[2], kc.shape[1]
    if out is None:
        out = _alloc_rows(q, T, Hq * D)
    args = (ptr(q), q.stride(0), ptr(kc), ptr(vc), max_seq, ptr(out), out.stride(0), T, p0, Hq, Hkv, D)
    if lse is None:
        check_rc(lib.hi_flash_prefill(*args, cur_stream()), "flash_prefill")
    else:
        check_rc(lib.hi_flash_prefill_lse(*args, ptr(lse), cur_stream()), "flash_prefill_lse")
    return out


def flash_prefill(q, kc, vc, T, p0, Hq, Hkv, out=None):
    """Causal attention for T prompt rows at positions p0.. of one cache slot: q [T, ldq] (head h at
    columns h*D), kc / vc [Hkv, max_seq, D]; returns [T, Hq*D] fp16."""
    return _flash(q, kc, vc, T, p0, Hq, Hkv, out, None)


def flash_prefill_lse(q, kc, vc, T, p0, Hq, Hkv, out=None, lse=None):
    """flash_prefill, also returning every (head, row)'s log-sum-exp of its scaled logits in base 2,
    lse [Hq, T] fp32: (out, lse)."""
    if lse is None:
        lse = torch.empty(Hq, T, dtype=torch.float32, device=q.device)
    _need("flash_prefill_lse", lse, torch.float32, 2)
    return _flash(q, kc, vc, T, p0, Hq, Hkv, out, lse), lse


def argmax(logits, out=None):
    """Greedy token of each row of logits [B, V] (NaN beats every number, the lowest index wins a tie,
    a row of -inf gives 0), as int32 [B]."""
    logits = logits.contiguous()
    _need("argmax", logits, torch.float16, 2)
    B, V = logits.shape
    if out is None:
        out = torch.empty(B, dtype=torch.int32, device=logits.device)
    check_rc(lib.hi_argmax(ptr(logits), B, V, ptr(out), cur_stream()), "argmax")
    return out


def embed(tok, table, out=None):
    """Embedding lookup: out[b] = table[tok[b]] for the int32 token ids tok [B]."""
    _need("embed", tok, torch.int32, 1)
    _need("embed", table, torch.float16, 2, rows=True)
    V, H = table.shape
    if out is None:
        out = _alloc_rows(table, tok.shape[0], H)
    check_rc(lib.hi_embed(ptr(tok), ptr(table), V, H, ptr(out), out.stride(0), tok.shape[0], cur_stream()), "embed")
    return out


# ------------------------------------------------------------------ int8 weight format
def quantize_rows(w):
    """Symmetric per-row int8 quantisation of fp16 weights w [N, K] on the GPU, bit for bit the
    reference exporter's: scale s[n] = fp16(max |w[n]| / 127), q = round-half-even(w / s) clamped to
    +-127 (an all-zero row gets q = 0). Returns (q int8 [N, K], s fp16 [N])."""
    _need("quantize_rows", w, torch.float16, 2)
    w = w.contiguous()
    N, K = w.shape
    q = torch.empty(N, K, dtype=torch.int8, device=w.device)
    s = torch.empty(N, dtype=torch.float16, device=w.device)
    check_rc(lib.hi_quantize_rows(ptr(w), N, K, ptr(q), ptr(s), cur_stream()), "quantize_rows")
    return q, s


def dequantize_rows(q, s):
    """The fp16 weights int8 rows stand for, fp16(q * s): what the prefill GEMM multiplies by."""
    _need("dequantize_rows", q, torch.int8, 2)
    _need("dequantize_rows", s, torch.float16, 1)
    q = q.contiguous()
    out = torch.empty(q.shape, dtype=torch.float16, device=q.device)
    check_rc(lib.hi_dequantize_rows(ptr(q), ptr(s), q.shape[0], q.shape[1], ptr(out), cur_stream()), "dequantize_rows")
    return out


def interleave_gate_up(gate, up, group=16):
    """The fused gate/up layout: for every block of `group` intermediate units, their gate rows
    followed by their up rows, [2I, H] from gate [I, H] and up [I, H] (any device or dtype)."""
    inter = gate.shape[0]
    if up.shape != gate.shape or inter % group:
        raise ValueError("hipinfer_amd.interleave_gate_up: gate and up must match, rows a multiple of the group")
    unit = torch.arange(inter, device=gate.device)
    # destination row of gate unit u: its group's first row, plus its place in the group
    dest = (unit // group) * (2 * group) + unit % group
    fused = gate.new_empty((2 * inter,) + tuple(gate.shape[1:]))
    fused[dest] = gate
    fused[dest + group] = up
    return fused


# ------------------------------------------------------------------ engine
def _ints(values):
    values = list(values)
    return (ctypes.c_int * max(1, len(values)))(*values), len(values)


class Engine:
    """A model from a weight file (the reference exporter's format: version 2 dense, 3 MoE, 4 int8)
    served on one GPU: max_batch cache slots of max_seq positions each, prompts prefilled in chunks
    of max_prefill rows, greedy decoding with the per-slot token history kept on the device.

    The reference's Engine API: prefill, prefill_logits, decode, history, logits, set_state, rewind,
    verify, generate, close, plus the model's shape as attributes. tp must be 1 (one GPU per engine;
    `devices`, if given, names it). A call the library rejects raises ValueError, with the reason on
    stderr."""

    MAX_VERIFY = lib.hi_verify_max_rows()  # draft rows per verify() call (k + 1 for k draft tokens)
    _CONFIG = ("vocab", "hidden", "inter", "layers", "heads", "kv_heads", "head_dim", "max_pos", "tied", "qkv_bias",
               "window")

    def __init__(self, path, max_batch=8, max_seq=2048, max_prefill=1024, tp=1, devices=None):
        if tp != 1:
            raise ValueError("hipinfer_amd.Engine: this build serves a model on one GPU (tp=1)")
        gpu = torch.cuda.current_device() if devices is None else int(list(devices)[0])
        self.tp, self.device = 1, torch.device("cuda", gpu)
        self.max_batch, self.max_seq, self.max_prefill = max_batch, max_seq, max_prefill
        devs, _ = _ints([gpu])
        self.h = lib.hi_load_tp(os.fsencode(path), max_batch, max_seq, max_prefill, 1, devs)
        if not self.h:
            raise RuntimeError(f"hipinfer_amd.Engine: loading {path} failed (reason on stderr)")
        fields = (ctypes.c_int * len(self._CONFIG))()
        lib.hi_config(self.h, fields)
        for name, value in zip(self._CONFIG, fields):
            setattr(self, name, bool(value) if name in ("tied", "qkv_bias") else value)
        moe = (ctypes.c_int * 3)()
        lib.hi_moe_config(self.h, moe)
        self.n_experts, self.top_k, self.moe_flags = moe  # zeros for a dense model
        self.quant = lib.hi_weight_quant(self.h)  # 0 fp16 projections, 1 int8 with fp16 row scales
        self.weight_bytes = lib.hi_weight_bytes(self.h)
        row = self.kv_heads * self.head_dim * 2  # one position's k (or v) in one layer, fp16
        self.kv_bytes_per_token = 2 * row * self.layers

    def _run(self, rc, what):
        if rc < 0:
            raise ValueError(f"hipinfer_amd.Engine.{what}: the library rejected the call (reason on stderr)")
        return rc

    def prefill(self, slot, tokens, p0=0):
        """Runs `tokens` through the model into cache slot `slot` at positions p0..; returns the greedy
        next token, which the slot will feed to its next decode step."""
        arr, n = _ints(tokens)
        return self._run(lib.hi_prefill(self.h, slot, arr, n, p0), "prefill")

    def prefill_logits(self, slot, tokens, p0=0):
        """prefill, returning the fp16 logits of every prompt position, [len(tokens), vocab] on the GPU."""
        arr, n = _ints(tokens)
        logits = torch.empty(n, self.vocab, dtype=torch.float16, device=self.device)
        self._run(lib.hi_prefill_logits(self.h, slot, arr, n, p0, ptr(logits)), "prefill_logits")
        return logits

    def decode(self, B, steps, graph=True):
        """`steps` greedy decode steps of slots 0..B-1 (replayed as a captured graph unless graph is
        False); returns the library's timing figure for the run."""
        return self._run(lib.hi_decode(self.h, B, steps, int(graph)), "decode")

    def history(self, slot, start, n):
        """Tokens at positions start .. start + n - 1 of a slot's history, as a list."""
        arr, _ = _ints([0] * n)
        self._run(lib.hi_history(self.h, slot, start, n, arr), "history")
        return list(arr)[:n]

    def logits(self, B):
        """The last decode step's logits of slots 0..B-1, [B, vocab] fp16 on the GPU."""
        out = torch.empty(B, self.vocab, dtype=torch.float16, device=self.device)
        self._run(lib.hi_logits(self.h, B, ptr(out)), "logits")
        return out

    def set_state(self, tokens, positions):
        """Sets slot i's next input token to tokens[i], fed at position positions[i]."""
        if len(tokens) != len(positions):
            raise ValueError("hipinfer_amd.Engine.set_state: one position per token")
        tok, B = _ints(tokens)
        pos, _ = _ints(positions)
        self._run(lib.hi_set_state(self.h, B, tok, pos), "set_state")

    def rewind(self, slot, length, next_token):
        """Truncates a slot to its first `length` cached positions; its next decode step feeds
        next_token at position `length`."""
        self._run(lib.hi_rewind(self.h, slot, length, next_token), "rewind")

    def verify(self, slot, tokens, p0, graph=True, logits=False):
        """Speculative verification of up to MAX_VERIFY rows: tokens[i] is fed at position p0 + i of
        `slot` (whose cache must already hold the positions before p0), all rows in one pass through
        the batch-of-one decode kernels, so entry i of the result is the token plain greedy decoding
        would emit after the same prefix, bit for bit. The rows' k / v stay in the cache; the slot's
        next token and position are not changed (rewind sets them after acceptance). Dense models.
        Returns the list of tokens, or (tokens, logits [R, vocab] fp16 on the GPU) with logits=True."""
        arr, R = _ints(tokens)
        picked = (ctypes.c_int * max(1, R))()
        lg = torch.empty(R, self.vocab, dtype=torch.float16, device=self.device) if logits else None
        self._run(lib.hi_verify(self.h, slot, arr, R, p0, picked, ptr(lg), int(graph)), "verify")
        toks = list(picked)[:R]
        return (toks, lg) if logits else toks

    def generate(self, prompt, n_new, graph=True):
        """Greedy continuation of `prompt` in slot 0: n_new token ids, the prefill's prediction first."""
        if n_new < 1:
            return []
        tokens = [self.prefill(0, prompt)]
        if n_new > 1:
            self.decode(1, n_new - 1, graph)
            tokens += self.history(0, len(prompt) + 1, n_new - 1)
        return tokens

    def close(self):
        """Frees the engine's GPU memory (idempotent)."""
        handle, self.h = getattr(self, "h", None), None
        if handle:
            lib.hi_free(handle)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
