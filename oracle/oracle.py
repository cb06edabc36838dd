"""ctypes wrapper of liboracle.so, the CPU oracle.  TEST INFRASTRUCTURE ONLY: imported by
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker; the product
(julia-cuda_amd/) never imports it.  See oracle.h for what each function restates."""

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

F32P = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
U16P = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
U32P = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
I32P = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")

# Tensor ids (oracle.h)
TOK_EMB, EMB_NORM, FINAL_NORM, TYPE_EMB = 1, 2, 3, 4
LAYER_BASE, HEAD_BASE, SCORER_BASE = 100, 1000, 2000
L_ATTN_NORM, L_WQKV, L_WO, L_MLP_NORM, L_WI, L_WO_MLP = range(6)
(H_NORM1_W, H_NORM1_B, H_IN_PROJ_W, H_IN_PROJ_B, H_OUT_PROJ_W, H_OUT_PROJ_B, H_NORM2_W,
 H_NORM2_B, H_LINEAR1_W, H_LINEAR1_B, H_LINEAR2_W, H_LINEAR2_B) = range(12)
S_NORM_W, S_NORM_B, S_LIN1_W, S_LIN1_B, S_LIN2_W, S_LIN2_B = range(6)

EPI_RES, EPI_GEGLU, EPI_LN, EPI_STATS, EPI_ROPE, EPI_BIAS, EPI_RELU, EPI_GELU = (
    1, 2, 4, 8, 16, 32, 64, 128)


class Cfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "d", "layers", "inter", "vocab", "head_layers", "head_ff", "n_qtypes", "window",
        "global_every", "max_positions")] + [
        (n, ctypes.c_float) for n in ("norm_eps", "head_eps", "theta_global", "theta_local")] + [
        ("seed", ctypes.c_uint64)]


def cfg(d=768, layers=22, inter=1152, vocab=50368, head_layers=2, head_ff=1536, n_qtypes=3,
        window=64, global_every=3, max_positions=8192, norm_eps=1e-5, head_eps=1e-5,
        theta_global=160000.0, theta_local=10000.0, seed=42):
    return Cfg(d, layers, inter, vocab, head_layers, head_ff, n_qtypes, window, global_every,
               max_positions, norm_eps, head_eps, theta_global, theta_local, seed)


def lib():
    global _LIB
    if _LIB is not None:
        return _LIB
    path = os.path.join(_HERE, "liboracle.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built (make -C oracle)")
    L = ctypes.CDLL(path)
    sig = {
        "oracle_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
        "oracle_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "oracle_round_f16": (None, [F32P, U16P, ctypes.c_size_t]),
        "oracle_gelu": (ctypes.c_float, [ctypes.c_float]),
        "oracle_synth": (None, [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_uint64,
                                ctypes.c_double, ctypes.c_double, F32P]),
        "oracle_tensor_dist": (ctypes.c_int, [ctypes.c_uint32, ctypes.POINTER(ctypes.c_double),
                                              ctypes.POINTER(ctypes.c_double)]),
        "oracle_fold_layernorm": (None, [F32P, F32P, ctypes.c_int, ctypes.c_int, U16P, F32P]),
        "oracle_fold_layernorm_bias": (None, [F32P, F32P, F32P, F32P, ctypes.c_int, ctypes.c_int,
                                              U16P, F32P, F32P]),
        "oracle_geglu_rows": (None, [ctypes.c_int, I32P]),
        "oracle_rope_table": (None, [ctypes.c_float, ctypes.c_int, F32P]),
        "oracle_layernorm_rows": (None, [F32P, F32P, ctypes.c_void_p, ctypes.c_float, ctypes.c_int,
                                         ctypes.c_int, F32P]),
        "oracle_linear": (None, [F32P, F32P, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int, F32P]),
        "oracle_rope_apply": (None, [F32P, ctypes.c_int, ctypes.c_int, F32P, ctypes.c_void_p]),
        "oracle_attention": (None, [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_int, F32P]),
        "oracle_geglu": (None, [F32P, ctypes.c_int, ctypes.c_int, F32P]),
        "oracle_row_stats": (None, [U16P, ctypes.c_int, ctypes.c_int, F32P]),
        "oracle_model_new": (ctypes.c_void_p, [ctypes.POINTER(Cfg)]),
        "oracle_model_free": (None, [ctypes.c_void_p]),
        "oracle_model_forward": (ctypes.c_int, [ctypes.c_void_p, U32P, ctypes.c_int, ctypes.c_int,
                                                U32P, ctypes.c_int, F32P, ctypes.c_void_p,
                                                ctypes.c_void_p]),
        "oracle_model_embed_rows": (None, [ctypes.c_void_p, U32P, ctypes.c_int, F32P]),
        "oracle_emu_embed": (None, [U16P, F32P, U32P, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                    U16P]),
        "oracle_emu_gemm": (None, [U16P, U16P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float,
                                   ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                   ctypes.c_int, U16P, ctypes.c_void_p]),
        "oracle_emu_attention": (None, [U16P, ctypes.c_int, ctypes.c_int, ctypes.c_int, U16P]),
        "oracle_emu_norm_add": (None, [U16P, F32P, F32P, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_float, U16P, F32P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _LIB = L
    return L


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u16(a):
    return np.ascontiguousarray(a, dtype=np.uint16)


# ---- numerics -----------------------------------------------------------------------------
def to_f16_bits(x):
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_round_f16(x.ravel(), out.ravel(), x.size)
    return out


def f16_bits_to_f32(h):
    return _u16(h).view(np.float16).astype(np.float32)


def gelu(x):
    return np.array([lib().oracle_gelu(float(v)) for v in np.ravel(x)], np.float32).reshape(np.shape(x))


# ---- synthetic weights --------------------------------------------------------------------
def dist(tid):
    m, s = ctypes.c_double(), ctypes.c_double()
    if lib().oracle_tensor_dist(tid, ctypes.byref(m), ctypes.byref(s)):
        raise KeyError(tid)
    return m.value, s.value


def synth(seed, tid, count, start=0, mean=None, std=None):
    if mean is None:
        mean, std = dist(tid)
    out = np.empty(count, np.float32)
    lib().oracle_synth(seed, tid, start, count, mean, std, out)
    return out


# ---- preparation --------------------------------------------------------------------------
def fold_layernorm(w, gamma):
    w, gamma = _f32(w), _f32(gamma)
    out, k = w.shape
    w16 = np.empty((out, k), np.uint16)
    cs = np.empty(out, np.float32)
    lib().oracle_fold_layernorm(w, gamma, out, k, w16, cs)
    return w16, cs


def fold_layernorm_bias(w, gamma, beta, b):
    w = _f32(w)
    out, k = w.shape
    w16 = np.empty((out, k), np.uint16)
    cs = np.empty(out, np.float32)
    bias = np.empty(out, np.float32)
    lib().oracle_fold_layernorm_bias(w, _f32(gamma), _f32(beta), _f32(b), out, k, w16, cs, bias)
    return w16, cs, bias


def geglu_rows(inter):
    src = np.empty(2 * inter, np.int32)
    lib().oracle_geglu_rows(inter, src)
    return src


def pack_frag(w16):
    """The GEMM kernels' weight order (a layout of this library's, no counterpart in the
    reference): w [n][k] as [n/64 groups][k/32 units][4 fragments][64 lanes][8], lane l holding
    row 64 G + 16 j + l % 16, columns 32 u + 8 (l / 16) + e. Restated with numpy axes, not
    by the library's loops."""
    w16 = np.asarray(w16)
    n, k = w16.shape
    return np.ascontiguousarray(
        w16.reshape(n // 64, 4, 16, k // 32, 4, 8).transpose(0, 3, 1, 4, 2, 5)).ravel()


def rope_table(theta, npos):
    t = np.empty((npos, 32, 2), np.float32)
    lib().oracle_rope_table(theta, npos, t)
    return t


# ---- f32 operations ---------------------------------------------------------------------
def layernorm_rows(x, gamma, beta=None, eps=1e-5):
    x = _f32(x)
    out = np.empty_like(x)
    b = None if beta is None else _f32(beta)
    lib().oracle_layernorm_rows(x, _f32(gamma), _ptr(b), eps, x.shape[0], x.shape[1], out)
    return out


def linear(x, w, b=None):
    x, w = _f32(x), _f32(w)
    y = np.empty((x.shape[0], w.shape[0]), np.float32)
    bb = None if b is None else _f32(b)
    lib().oracle_linear(x, w, _ptr(bb), x.shape[0], x.shape[1], w.shape[0], y)
    return y


def rope_apply(qkv, table, pos=None):
    qkv = _f32(qkv).copy()
    n, d3 = qkv.shape
    p = None if pos is None else np.ascontiguousarray(pos, np.int32)
    lib().oracle_rope_apply(qkv, n, d3 // 3, _f32(table), _ptr(p))
    return qkv


def attention(qkv, window=0):
    """Attention over a [n, 3d] qkv (heads of 64) in f64; returns [n, d]."""
    qkv = _f32(qkv)
    n, d3 = qkv.shape
    d = d3 // 3
    o = np.empty((n, d), np.float32)
    base = qkv.ctypes.data
    lib().oracle_attention(ctypes.c_void_p(base), d3, ctypes.c_void_p(base + 4 * d), d3, n, d,
                           window, o)
    return o


def geglu(hh):
    hh = _f32(hh)
    m = np.empty((hh.shape[0], hh.shape[1] // 2), np.float32)
    lib().oracle_geglu(hh, hh.shape[0], hh.shape[1] // 2, m)
    return m


def row_stats(x16):
    x16 = _u16(x16)
    rows, k = x16.shape
    st = np.empty((rows, k // 64, 2), np.float32)
    lib().oracle_row_stats(x16, rows, k, st)
    return st


# ---- the model ----------------------------------------------------------------------------
class Model:
    """The synthetic Julia-1-shaped model, f32, unfolded weights."""

    def __init__(self, c):
        self.cfg = c
        self.ptr = lib().oracle_model_new(ctypes.byref(c))
        if not self.ptr:
            raise ValueError("oracle_model_new failed")

    def __del__(self):
        if getattr(self, "ptr", None):
            lib().oracle_model_free(self.ptr)
            self.ptr = None

    def forward(self, ids, qtype, markers, trace=False, head_x=False):
        ids = np.ascontiguousarray(ids, np.uint32)
        markers = np.ascontiguousarray(markers, np.uint32)
        n, d = len(ids), self.cfg.d
        logits = np.empty(max(len(markers), 1), np.float32)
        xt = np.empty((self.cfg.layers, n, d), np.float32) if trace else None
        hx = np.empty((n, d), np.float32) if head_x else None
        rc = lib().oracle_model_forward(self.ptr, ids, n, qtype, markers, len(markers), logits,
                                        _ptr(xt), _ptr(hx))
        if rc:
            raise ValueError("oracle_model_forward rejected its arguments")
        out = [logits[: len(markers)]]
        if trace:
            out.append(xt)
        if head_x:
            out.append(hx)
        return out[0] if len(out) == 1 else tuple(out)

    def embed_rows(self, ids):
        ids = np.ascontiguousarray(ids, np.uint32)
        out = np.empty((len(ids), self.cfg.d), np.float32)
        lib().oracle_model_embed_rows(self.ptr, ids, len(ids), out)
        return out


# ---- f16 emulation ------------------------------------------------------------------------
def emu_embed(table16, gamma, ids, eps=1e-5):
    table16 = _u16(table16)
    ids = np.ascontiguousarray(ids, np.uint32)
    d = table16.shape[1]
    x = np.empty((len(ids), d), np.uint16)
    lib().oracle_emu_embed(table16, _f32(gamma), ids, len(ids), d, eps, x)
    return x


def emu_gemm(a16, w16, epi, stats_in=None, colsum=None, eps=1e-5, bias=None, rope=None,
             pos=None, rope_cols=0, c16=None):
    a16, w16 = _u16(a16), _u16(w16)
    m, k = a16.shape
    n = w16.shape[0]
    ncols = n // 2 if epi & EPI_GEGLU else n
    c = np.zeros((m, ncols), np.uint16) if c16 is None else _u16(c16).copy()
    st_out = np.zeros((m, n // 64, 2), np.float32) if epi & EPI_STATS else None
    si = None if stats_in is None else _f32(stats_in)
    cs = None if colsum is None else _f32(colsum)
    b = None if bias is None else _f32(bias)
    r = None if rope is None else _f32(rope)
    p = None if pos is None else np.ascontiguousarray(pos, np.int32)
    lib().oracle_emu_gemm(a16, w16, m, n, k, epi, _ptr(si), _ptr(cs), eps, _ptr(b), _ptr(r),
                          _ptr(p), rope_cols, c, _ptr(st_out))
    return (c, st_out) if epi & EPI_STATS else c


def emu_attention(qkv16, window=0):
    qkv16 = _u16(qkv16)
    n, d3 = qkv16.shape
    o = np.empty((n, d3 // 3), np.uint16)
    lib().oracle_emu_attention(qkv16, n, d3 // 3, window, o)
    return o


def emu_norm_add(x16, gamma, add, eps=1e-5):
    x16 = _u16(x16)
    n, d = x16.shape
    out = np.empty((n, d), np.uint16)
    st = np.empty((n, d // 64, 2), np.float32)
    lib().oracle_emu_norm_add(x16, _f32(gamma), _f32(add), n, d, eps, out, st)
    return out, st


# ---- error measures (src/check.rs:38-60) -------------------------------------------------
def rel_err(a, b):
    """Frobenius relative error ||a - b|| / ||b||, in f64 (src/check.rs:38-46)."""
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.sqrt(np.sum((a - b) ** 2) / np.sum(b ** 2)))


def max_rel(a, b):
    """max |a - b| / max |b|: the element-wise bound the north-star tolerance is stated in."""
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def ulps(a16, b16):
    """f16 steps between two bit patterns, +-0 equal (src/check.rs:48-60)."""
    def ordered(x):
        x = np.asarray(x, np.uint16).astype(np.int32)
        return np.where(x & 0x8000, -(x & 0x7FFF), x)
    return np.abs(ordered(a16) - ordered(b16))
