"""The CPU oracle for zwhisper's attention hot path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package,
and only as the checker (or, in bench.py, as the timed CPU baseline).  The product — the HIP
library under zwhisper_amd/ — never imports, links or calls anything here.

Contents:
* ``Oracle``: ctypes front end to liboracle_v{3,4}.so, the C restatement of the reference's
  ops.attentionEx / attention / pvBlock / expVec / softmaxRow / Pool, and ops.linear with f16
  weights (gemm.ntBlock) or int8 block weights (gemm.Q8, Q8.quantize, ntBlockQ)
  (oracle/attn_oracle.c, which cites src/ops.zig and src/gemm.zig line by line).
* ``naive``: the f64 closed form (oracle/naive.py).
* ``kv``: the reference's cache writes -- rotary tables and NeoX rotation, the transposed key
  scatter, row appends (oracle/kv.py, citing src/llm.zig and src/decoder.zig).

Parity pinning of each function lives in tests/test_oracle.py and tests/test_kv_oracle.py.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from . import naive  # noqa: F401

_HERE = os.path.dirname(os.path.abspath(__file__))
_c_size = ctypes.c_size_t
_fp = ctypes.POINTER(ctypes.c_float)

V = 16
Q_BLOCK = 64


class OraShape(ctypes.Structure):
    """Mirror of AttnShape (src/ops.zig:477-492); kt_stride 0 stands for null."""

    _fields_ = [
        ("n_q", ctypes.c_uint64),
        ("n_kv", ctypes.c_uint64),
        ("n_head", ctypes.c_uint64),
        ("n_head_kv", ctypes.c_uint64),
        ("d", ctypes.c_uint64),
        ("q_stride", ctypes.c_uint64),
        ("kv_stride", ctypes.c_uint64),
        ("out_stride", ctypes.c_uint64),
        ("kt_stride", ctypes.c_uint64),
        ("causal", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
    ]


def _host_has_avx512() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
                    return {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"} <= flags
    except OSError:
        pass
    return False


def build() -> None:
    """Compile liboracle_v3.so / liboracle_v4.so from attn_oracle.c (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", _HERE, "-j2"], check=True)


def library_path() -> str:
    return os.path.join(_HERE, "liboracle_v4.so" if _host_has_avx512() else "liboracle_v3.so")


_lib = None


def lib():
    global _lib
    if _lib is None:
        path = library_path()
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        L.ora_pool_new.restype = ctypes.c_void_p
        L.ora_pool_new.argtypes = [_c_size]
        L.ora_pool_free.argtypes = [ctypes.c_void_p]
        L.ora_pool_size.restype = _c_size
        L.ora_pool_size.argtypes = [ctypes.c_void_p]
        L.ora_attention_ex.restype = ctypes.c_int
        L.ora_attention_ex.argtypes = [ctypes.c_void_p, _fp, _fp, _fp, ctypes.POINTER(OraShape), _fp, _c_size, _fp]
        L.ora_attention.restype = ctypes.c_int
        L.ora_attention.argtypes = [ctypes.c_void_p, _fp, _fp, _fp, _c_size, _c_size, _c_size, _c_size, ctypes.c_int,
                                    _fp, _c_size, _fp]
        for name in ("ora_attention_scratch_ex",):
            getattr(L, name).restype = _c_size
            getattr(L, name).argtypes = [_c_size] * 5
        L.ora_attention_scratch_kt.restype = _c_size
        L.ora_attention_scratch_kt.argtypes = [_c_size] * 3
        L.ora_attention_scratch.restype = _c_size
        L.ora_attention_scratch.argtypes = [_c_size] * 4
        L.ora_exp_vec.argtypes = [_fp, _fp, _c_size]
        L.ora_softmax_row.argtypes = [_fp, _c_size]
        L.ora_pv_block.argtypes = [_fp, _c_size, _fp, _c_size, _fp, _c_size, _c_size, _c_size, _c_size]
        L.ora_vector_width.restype = ctypes.c_int
        L.ora_q_block.restype = ctypes.c_int
        L.ora_linear_f16.restype = None
        L.ora_linear_f16.argtypes = [ctypes.c_void_p, _fp, _c_size, _c_size, ctypes.c_void_p, ctypes.c_void_p, _c_size,
                                     _fp]
        L.ora_linear_q8.restype = None
        L.ora_linear_q8.argtypes = [ctypes.c_void_p, _fp, _c_size, _c_size, ctypes.c_void_p, _fp, ctypes.c_void_p,
                                    _c_size, _fp]
        L.ora_layer_norm.restype = None
        L.ora_layer_norm.argtypes = [ctypes.c_void_p, _fp, _c_size, _c_size, _fp, _fp, ctypes.c_float, _fp]
        L.ora_gelu.restype = None
        L.ora_gelu.argtypes = [ctypes.c_void_p, _fp, _c_size]
        L.ora_rms_norm.restype = None
        L.ora_rms_norm.argtypes = [_fp, _c_size, _c_size, _fp, ctypes.c_float, _fp]
        L.ora_silu_mul.restype = None
        L.ora_silu_mul.argtypes = [_fp, _fp, _c_size]
        L.ora_q8_quantize.restype = None
        L.ora_q8_quantize.argtypes = [_fp, _c_size, _c_size, ctypes.c_void_p, _fp]
        _lib = L
    return _lib


Q8_BLOCK = 32


def q8_quantize(w, n: int, k: int):
    """gemm.Q8.quantize (src/gemm.zig:209-230) of an [n][k] f16 or f32 matrix: (q int8 [n][k],
    scales f32 [n][k / 32])."""
    if k % Q8_BLOCK:
        raise ValueError("k must be a multiple of 32")
    w = np.ascontiguousarray(np.asarray(w).reshape(-1)[: n * k], dtype=np.float32)
    q = np.zeros(n * k, np.int8)
    sc = np.zeros(n * (k // Q8_BLOCK), np.float32)
    lib().ora_q8_quantize(_ptr(w), n, k, q.ctypes.data, _ptr(sc))
    return q.reshape(n, k), sc.reshape(n, k // Q8_BLOCK)


def q8_dequantize(q, scales) -> np.ndarray:
    """Q8.row (src/gemm.zig:255-263) for every row: f32(q) * scale, [n][k]."""
    q = np.asarray(q, dtype=np.int8)
    n, k = q.shape
    return (q.reshape(n, k // Q8_BLOCK, Q8_BLOCK).astype(np.float32)
            * np.asarray(scales, np.float32).reshape(n, -1, 1)).reshape(n, k)


def _ptr(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_fp)


def _check_lengths(q, k, v, out, sh) -> None:
    """The C code trusts its buffers: refuse arrays shorter than the shape reads or writes."""
    kvd = sh.n_head_kv * sh.d
    need_q = (sh.n_q - 1) * sh.q_stride + sh.n_head * sh.d if sh.n_q else 0
    need_o = (sh.n_q - 1) * sh.out_stride + sh.n_head * sh.d if sh.n_q else 0
    if sh.n_kv == 0:
        need_k = need_v = 0
    elif sh.kt_stride:
        # the reference reads round_up(n_kv, V) columns of every transposed row
        need_k = (kvd - 1) * sh.kt_stride + (sh.n_kv + V - 1) // V * V
        need_v = (sh.n_kv - 1) * sh.kv_stride + kvd
    else:
        need_k = need_v = (sh.n_kv - 1) * sh.kv_stride + kvd
    for name, arr, need in (("q", q, need_q), ("k", k, need_k), ("v", v, need_v), ("out", out, need_o)):
        if arr.size < need:
            raise ValueError(f"{name} holds {arr.size} floats, the shape needs {need}")


def to_ora_shape(sh) -> OraShape:
    return OraShape(sh.n_q, sh.n_kv, sh.n_head, sh.n_head_kv, sh.d, sh.q_stride, sh.kv_stride, sh.out_stride,
                    sh.kt_stride or 0, 1 if sh.causal else 0, 0)


def scratch_floats(sh) -> int:
    L = lib()
    if sh.kt_stride:
        return int(L.ora_attention_scratch_kt(sh.n_q, sh.kt_stride, sh.n_head))
    return int(L.ora_attention_scratch_ex(sh.n_q, sh.n_kv, sh.n_head, sh.n_head_kv, sh.d))


class Oracle:
    """The reference's multithreaded f32 attention, restated in C, with its own Pool."""

    def __init__(self, threads: int = 1):
        self._L = lib()
        self._pool = self._L.ora_pool_new(max(1, int(threads)))
        self.threads = int(self._L.ora_pool_size(self._pool))

    def close(self) -> None:
        if self._pool:
            self._L.ora_pool_free(self._pool)
            self._pool = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def attention_ex(self, q, k, v, sh, out=None, scratch=None) -> np.ndarray:
        """ops.attentionEx on numpy f32 buffers; returns out (flat, [n_q][out_stride])."""
        q = np.ascontiguousarray(q, dtype=np.float32).reshape(-1)
        k = np.ascontiguousarray(k, dtype=np.float32).reshape(-1)
        v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1)
        n_out = (sh.n_q - 1) * sh.out_stride + sh.n_head * sh.d if sh.n_q else 0
        if out is None:
            out = np.zeros(max(n_out, 1), dtype=np.float32)
        _check_lengths(q, k, v, out, sh)
        if scratch is None:
            scratch = np.empty(max(scratch_floats(sh), 1), dtype=np.float32)
        shape = to_ora_shape(sh)
        rc = self._L.ora_attention_ex(self._pool, _ptr(q), _ptr(k), _ptr(v), ctypes.byref(shape), _ptr(scratch),
                                      scratch.size, _ptr(out))
        if rc != 0:
            raise ValueError(f"oracle rejected shape {sh}")
        return out

    def linear_f16(self, x, m: int, k: int, w, b, n: int, out=None) -> np.ndarray:
        """ops.linear with f16 weights (src/ops.zig:283-306): x f32 [m][k], w float16 [n][k], b f32 [n] or None."""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        w = np.ascontiguousarray(w, dtype=np.float16).reshape(-1)
        if x.size < m * k or w.size < n * k:
            raise ValueError("x or w shorter than m*k / n*k")
        bb = None if b is None else np.ascontiguousarray(b, dtype=np.float32).reshape(-1)
        if out is None:
            out = np.zeros(max(m * n, 1), dtype=np.float32)
        self._L.ora_linear_f16(self._pool, _ptr(x), m, k, w.ctypes.data, None if bb is None else bb.ctypes.data, n,
                               _ptr(out))
        return out

    def linear_q8(self, x, m: int, k: int, q, scales, b, n: int, out=None) -> np.ndarray:
        """ops.linear with gemm.Q8 weights (src/ops.zig:283-306, src/gemm.zig:336-351): q int8
        [n][k], scales f32 [n][k / 32], k a multiple of 32."""
        if k % Q8_BLOCK:
            raise ValueError("k must be a multiple of 32")
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        q = np.ascontiguousarray(q, dtype=np.int8).reshape(-1)
        sc = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
        if x.size < m * k or q.size < n * k or sc.size < n * (k // Q8_BLOCK):
            raise ValueError("x, q or scales shorter than the shape needs")
        bb = None if b is None else np.ascontiguousarray(b, dtype=np.float32).reshape(-1)
        if out is None:
            out = np.zeros(max(m * n, 1), dtype=np.float32)
        self._L.ora_linear_q8(self._pool, _ptr(x), m, k, q.ctypes.data, _ptr(sc),
                              None if bb is None else bb.ctypes.data, n, _ptr(out))
        return out

    def layer_norm(self, x, m: int, n: int, w, b, eps: float = 1e-5) -> np.ndarray:
        """ops.layerNormEps (src/ops.zig:388-395) of x [m][n]; returns out [m][n]."""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
        b = np.ascontiguousarray(b, dtype=np.float32).reshape(-1)
        if x.size < m * n or w.size < n or b.size < n:
            raise ValueError("x, w or b shorter than the shape needs")
        out = np.empty(m * n, np.float32)
        self._L.ora_layer_norm(self._pool, _ptr(x), m, n, _ptr(w), _ptr(b), eps, _ptr(out))
        return out.reshape(m, n)

    def gelu(self, x) -> np.ndarray:
        """ops.gelu (src/ops.zig:335-340) on a copy of x."""
        y = np.ascontiguousarray(x, dtype=np.float32).copy()
        self._L.ora_gelu(self._pool, _ptr(y.reshape(-1)), y.size)
        return y

    def rms_norm(self, x, m: int, n: int, w, eps: float) -> np.ndarray:
        """ops.rmsNorm (src/ops.zig:409-427) of x [m][n]; returns out [m][n]."""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
        if x.size < m * n or w.size < n:
            raise ValueError("x or w shorter than the shape needs")
        out = np.empty(m * n, np.float32)
        self._L.ora_rms_norm(_ptr(x), m, n, _ptr(w), eps, _ptr(out))
        return out.reshape(m, n)

    def silu_mul(self, gate, up) -> np.ndarray:
        """ops.siluMul (src/ops.zig:435-439) on a copy of gate: gate / (1 + e^-gate) * up."""
        g = np.ascontiguousarray(gate, dtype=np.float32).copy()
        u = np.ascontiguousarray(up, dtype=np.float32).reshape(-1)
        if u.size < g.size:
            raise ValueError("up shorter than gate")
        self._L.ora_silu_mul(_ptr(g.reshape(-1)), _ptr(u), g.size)
        return g

    def encoder_layer(self, x, n_ctx: int, n_state: int, n_head: int, w: dict) -> np.ndarray:
        """One Whisper encoder layer (src/encoder.zig:164-175) on one window x [n_ctx][n_state] with f16
        weights (w: attn_ln_w/b, q_w/q_b, k_w, v_w/v_b, o_w/o_b, mlp_ln_w/b, mlp0_w/b, mlp1_w/b); returns
        the new x.  ops.add is the plain f32 sum."""
        ns = n_state
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(n_ctx, ns).copy()
        xl = self.layer_norm(x, n_ctx, ns, w["attn_ln_w"], w["attn_ln_b"])
        q = self.linear_f16(xl, n_ctx, ns, w["q_w"], w["q_b"], ns)
        k = self.linear_f16(xl, n_ctx, ns, w["k_w"], None, ns)
        v = self.linear_f16(xl, n_ctx, ns, w["v_w"], w["v_b"], ns)
        att = self.attention(q, k, v, n_ctx, n_ctx, ns, n_head, False)
        x += self.linear_f16(att, n_ctx, ns, w["o_w"], w["o_b"], ns).reshape(n_ctx, ns)
        xl = self.layer_norm(x, n_ctx, ns, w["mlp_ln_w"], w["mlp_ln_b"])
        h = self.gelu(self.linear_f16(xl, n_ctx, ns, w["mlp0_w"], w["mlp0_b"], 4 * ns))
        x += self.linear_f16(h, n_ctx, 4 * ns, w["mlp1_w"], w["mlp1_b"], ns).reshape(n_ctx, ns)
        return x

    def decoder_set_audio(self, enc, n_audio_ctx: int, n_state: int, layers) -> list:
        """Decoder.setAudio (src/decoder.zig:151-159) for one window: per layer (cross_k, cross_v)
        [n_audio_ctx][n_state] = enc . ck^T and enc . cv^T + cv_b.  Matrices are (q, scales) pairs
        of gemm.Q8 (int8 [n][k], f32 [n][k / 32])."""
        ns = n_state
        out = []
        for w in layers:
            ck = self.linear_q8(enc, n_audio_ctx, ns, *w["ck_w"], None, ns).reshape(n_audio_ctx, ns)
            cv = self.linear_q8(enc, n_audio_ctx, ns, *w["cv_w"], w["cv_b"], ns).reshape(n_audio_ctx, ns)
            out.append((ck, cv))
        return out

    def decoder_forward(self, dec: dict, cache: dict, token: int, pos: int) -> np.ndarray:
        """Decoder.forward (src/decoder.zig:165-205) for one window and one token at position pos
        (n_past), as the reference runs it: x = te.row(token) + pe[pos] (src/gemm.zig:257-265,
        ops.add); per layer the pre-norm self-attention over the cache (k and v rows written at pos,
        then attention causal over pos + 1 keys), the cross-attention over the window's cross K/V
        and the MLP, each added to x; then the final layer norm and logits = ln(x) . te^T.
        dec: {"te": (q, scales) [n_vocab][n_state], "pe", "ln_w", "ln_b", "n_head", "layers": [dict
        of the layer's tensors, matrices as (q, scales)]}; cache: {"k", "v": [n_layer][n_ctx][ns],
        "ck", "cv": [n_layer][n_audio_ctx][ns]} (k and v updated at row pos).  Returns the logits."""
        te_q, te_s = dec["te"]
        n_vocab, ns = te_q.shape
        H = dec["n_head"]
        lin = lambda a, w, b, n, k: self.linear_q8(a, 1, k, *w, b, n)  # noqa: E731
        row = te_q[token].astype(np.float32).reshape(-1, Q8_BLOCK) * te_s[token].astype(np.float32)[:, None]
        x = (row.reshape(-1) + dec["pe"][pos]).astype(np.float32)
        n_audio = cache["ck"].shape[1]
        for li, w in enumerate(dec["layers"]):
            xl = self.layer_norm(x, 1, ns, w["attn_ln_w"], w["attn_ln_b"])
            q = lin(xl, w["q_w"], w["q_b"], ns, ns)
            cache["k"][li][pos] = lin(xl, w["k_w"], None, ns, ns)
            cache["v"][li][pos] = lin(xl, w["v_w"], w["v_b"], ns, ns)
            att = self.attention(q, cache["k"][li][:pos + 1], cache["v"][li][:pos + 1], 1, pos + 1, ns, H, True)
            x = x + lin(att, w["o_w"], w["o_b"], ns, ns)
            xl = self.layer_norm(x, 1, ns, w["cross_ln_w"], w["cross_ln_b"])
            q = lin(xl, w["cq_w"], w["cq_b"], ns, ns)
            att = self.attention(q, cache["ck"][li], cache["cv"][li], 1, n_audio, ns, H, False)
            x = x + lin(att, w["co_w"], w["co_b"], ns, ns)
            xl = self.layer_norm(x, 1, ns, w["mlp_ln_w"], w["mlp_ln_b"])
            h = self.gelu(lin(xl, w["mlp0_w"], w["mlp0_b"], 4 * ns, ns))
            x = x + lin(h, w["mlp1_w"], w["mlp1_b"], ns, 4 * ns)
        xl = self.layer_norm(x, 1, ns, dec["ln_w"], dec["ln_b"])
        return self.linear_q8(xl, 1, ns, te_q, te_s, None, n_vocab)

    def llm_forward(self, lm: dict, cache: dict, token, pos: int) -> np.ndarray:
        """Model.forward (src/llm.zig:169-216) for one sequence and one token, or a list of n
        tokens, at positions pos .. pos + n - 1 (n_past = pos), as the reference runs it: x =
        embd.row(token) per row; per layer rmsNorm, q/k/v with their biases, NeoX rotary positions
        on q and k, k scattered into the transposed cache and v into its rows (oracle/kv.py
        llm_append), attentionEx over the pos + n cached keys (causal, kt_stride = n_ctx), o added
        into x, rmsNorm, the SiLU-gated MLP added into x; then the output norm of the last row and
        its logits = norm(x) . output^T.  lm: {"embd": (q, scales), "output": (q, scales),
        "output_norm", "n_head", "n_head_kv", "eps", "cos", "sin", "layers": [dict of the layer's
        tensors, matrices as (q, scales)]}; cache: {"kt": [n_layer][n_head_kv * d * n_ctx], "v":
        [n_layer][n_ctx][n_head_kv * d]} (updated at pos ..).  Returns the last token's logits."""
        from types import SimpleNamespace

        from . import kv as kvo

        toks = [int(token)] if np.ndim(token) == 0 else [int(t) for t in token]
        n = len(toks)
        e_q, e_s = lm["embd"]
        n_vocab, ne = e_q.shape
        H, Hk, eps = lm["n_head"], lm["n_head_kv"], lm["eps"]
        d = ne // H
        kvw = Hk * d
        n_ctx = cache["v"].shape[1]
        lin = lambda a, w, b, nn, k: self.linear_q8(a, n, k, *w, b, nn)  # noqa: E731
        x = np.concatenate([(e_q[t].astype(np.float32).reshape(-1, Q8_BLOCK) *
                             e_s[t].astype(np.float32)[:, None]).reshape(-1) for t in toks])
        for li, w in enumerate(lm["layers"]):
            h = self.rms_norm(x, n, ne, w["attn_norm"], eps)
            q = lin(h, w["wq"], w.get("bq"), ne, ne)
            k = lin(h, w["wk"], w.get("bk"), kvw, ne)
            v = lin(h, w["wv"], w.get("bv"), kvw, ne)
            kvo.llm_append(q, k, v, n, pos, H, Hk, d, ne, cache["kt"][li], cache["v"][li], n_ctx, lm["cos"], lm["sin"])
            sh = SimpleNamespace(n_q=n, n_kv=pos + n, n_head=H, n_head_kv=Hk, d=d, q_stride=ne, kv_stride=kvw,
                                 out_stride=ne, causal=True, kt_stride=n_ctx)
            att = self.attention_ex(q, cache["kt"][li], cache["v"][li][:pos + n], sh)
            x = x + lin(att, w["wo"], None, ne, ne)
            h = self.rms_norm(x, n, ne, w["ffn_norm"], eps)
            nff = w["w_gate"][0].shape[0]
            g = lin(h, w["w_gate"], None, nff, ne)
            u = lin(h, w["w_up"], None, nff, ne)
            g = self.silu_mul(g, u)
            x = x + lin(g, w["w_down"], None, ne, nff)
        h = self.rms_norm(x[(n - 1) * ne:], 1, ne, lm["output_norm"], eps)
        return self.linear_q8(h, 1, ne, *lm["output"], None, n_vocab)

    def attention(self, q, k, v, n_q, n_kv, n_state, n_head, causal, out=None) -> np.ndarray:
        """ops.attention (src/ops.zig:593-605)."""
        q = np.ascontiguousarray(q, dtype=np.float32).reshape(-1)
        k = np.ascontiguousarray(k, dtype=np.float32).reshape(-1)
        v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1)
        if out is None:
            out = np.zeros(max(n_q * n_state, 1), dtype=np.float32)
        if q.size < n_q * n_state or k.size < n_kv * n_state or v.size < n_kv * n_state or out.size < n_q * n_state:
            raise ValueError("a buffer is shorter than n_q/n_kv x n_state")
        scratch = np.empty(max(int(self._L.ora_attention_scratch(n_q, n_kv, n_head, n_state)), 1), dtype=np.float32)
        rc = self._L.ora_attention(self._pool, _ptr(q), _ptr(k), _ptr(v), n_q, n_kv, n_state, n_head,
                                   1 if causal else 0, _ptr(scratch), scratch.size, _ptr(out))
        if rc != 0:
            raise ValueError("oracle rejected shape")
        return out


def exp_vec(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.size % V == 0
    y = np.empty_like(x)
    lib().ora_exp_vec(_ptr(x), _ptr(y), x.size)
    return y


def softmax_row(x: np.ndarray) -> np.ndarray:
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    lib().ora_softmax_row(_ptr(y), y.size)
    return y


def pv_block(p: np.ndarray, v: np.ndarray) -> np.ndarray:
    """C[m][d] = P[m][t] . V[t][d] (gemm.pvBlock)."""
    p = np.ascontiguousarray(p, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    m, t = p.shape
    t2, d = v.shape
    assert t == t2 and d % V == 0
    c = np.empty((m, d), dtype=np.float32)
    lib().ora_pv_block(_ptr(p), t, _ptr(v), d, _ptr(c), d, m, t, d)
    return c
