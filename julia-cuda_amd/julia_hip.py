"""ctypes binding of libjulia_hip.so (include/julia_hip.h), the way the reference's callers bind
its C interface (src/capi.rs:1-2: megaLaya's harness loads the library with ctypes).

`Engine` mirrors src/capi.rs (julia_cuda_load / run / free / device / tier); the op functions
mirror the reference's internal per-op surface (gemm::launch, attn::launch, embed_into, ...) on
caller-owned device memory: pass device addresses (e.g. torch.Tensor.data_ptr()) and a HIP
stream handle (torch.cuda.current_stream().cuda_stream), or 0 for the null stream.

The library must be built (`make -C julia-cuda_amd`); there is no fallback.
"""

import ctypes
import os
import sys

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libjulia_hip.so")
_LIB = None

EPI_RES, EPI_GEGLU, EPI_LN, EPI_STATS, EPI_ROPE, EPI_BIAS, EPI_RELU, EPI_GELU = (
    1, 2, 4, 8, 16, 32, 64, 128)
EPI = {
    "rope": EPI_ROPE,
    "lnrope": EPI_LN | EPI_ROPE,
    "lngeglu": EPI_LN | EPI_GEGLU,
    "resstats": EPI_RES | EPI_STATS,
    "lnbias": EPI_LN | EPI_BIAS,
    "lnbiasrelu": EPI_LN | EPI_BIAS | EPI_RELU,
    "lnbiasgelu": EPI_LN | EPI_BIAS | EPI_GELU,
    "biasresstats": EPI_BIAS | EPI_RES | EPI_STATS,
}

ERR_LEN = 1024
PROF_WORDS = 32  # u64 stamps per block and layer of the persistent kernel's profile


class JuliaHipError(RuntimeError):
    pass


class GemmArgs(ctypes.Structure):
    _fields_ = [
        ("epi", ctypes.c_int),
        ("a", ctypes.c_void_p),
        ("w", ctypes.c_void_p),
        ("c", ctypes.c_void_p),
        ("m", ctypes.c_int),
        ("n", ctypes.c_int),
        ("k", ctypes.c_int),
        ("stats_in", ctypes.c_void_p),
        ("colsum", ctypes.c_void_p),
        ("eps", ctypes.c_float),
        ("bias", ctypes.c_void_p),
        ("rope", ctypes.c_void_p),
        ("positions", ctypes.c_void_p),
        ("rope_rows", ctypes.c_int),
        ("stats_out", ctypes.c_void_p),
    ]


class GemmConfig(ctypes.Structure):
    _fields_ = [("bm", ctypes.c_int), ("splits", ctypes.c_int)]

    def __repr__(self):
        return f"GemmConfig(bm={self.bm}, splits={self.splits})"


class EngineInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "d", "layers", "inter", "vocab", "head_layers", "head_ff", "n_qtypes", "window",
        "global_every", "max_positions", "max_length", "cus")] + [
        ("norm_eps", ctypes.c_float), ("head_eps", ctypes.c_float), ("seed", ctypes.c_uint64),
        ("weight_bytes_f16", ctypes.c_size_t), ("weight_bytes_f32", ctypes.c_size_t),
        ("coop_refused", ctypes.c_size_t)]


# Every symbol include/julia_hip.h declares.
EXPORTS = [
    "julia_cuda_tier", "julia_cuda_load", "julia_cuda_free", "julia_cuda_device", "julia_cuda_run",
    "julia_hip_load", "julia_hip_run_batched", "julia_hip_model_kernel",
    "julia_hip_scratch_new", "julia_hip_scratch_free", "julia_hip_gemm", "julia_hip_gemm_static",
    "julia_hip_attention",
    "julia_hip_attention_seg",
    "julia_hip_embed", "julia_hip_norm_add", "julia_hip_score", "julia_hip_time_gemm",
    "julia_hip_time_attention", "julia_hip_time_copy", "julia_hip_copy", "julia_hip_device_count",
    "julia_hip_device_alloc", "julia_hip_device_free", "julia_hip_device_sync",
    "julia_hip_prep_fold_layernorm", "julia_hip_prep_fold_layernorm_bias",
    "julia_hip_prep_geglu_rows", "julia_hip_prep_pack_frag", "julia_hip_prep_unpack_frag",
    "julia_hip_prep_rope_table", "julia_hip_synth",
    "julia_hip_round_f16", "julia_hip_gemm_choose", "julia_hip_gemm_check", "julia_hip_gemm_plan_2080ti",
    "julia_hip_gemm_choose_2080ti", "julia_hip_engine_info_get", "julia_hip_engine_tensor",
    "julia_hip_time_encoder_step", "julia_hip_profile_layer", "julia_hip_run_trace",
    "julia_hip_encode_batch",
    "julia_hip_encode_batch_phases", "julia_hip_checkpoint_config", "julia_hip_answer",
    "julia_hip_latency_summary",
]

_VP, _SZ, _I, _F, _CP = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_float, ctypes.c_char_p
_F32P = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_U16P = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_I32P = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_F64P = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")


def lib():
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise JuliaHipError(f"{LIB_PATH} is not built: run `make -C julia-cuda_amd`")
    L = ctypes.CDLL(LIB_PATH)
    sig = {
        "julia_cuda_tier": (_CP, []),
        "julia_cuda_load": (_VP, [_CP, _SZ, _CP, _SZ]),
        "julia_cuda_free": (None, [_VP]),
        "julia_cuda_device": (None, [_VP, _CP, _SZ]),
        "julia_cuda_run": (_I, [_VP, _SZ, _VP, _VP, _VP, _VP, _VP, _I, _VP, _VP, _CP, _SZ]),
        "julia_hip_load": (_VP, [_CP, _SZ, _SZ, _CP, _SZ]),
        "julia_hip_model_kernel": (_I, [_VP, _SZ]),
        "julia_hip_run_batched": (_I, [_VP, _SZ, _VP, _VP, _VP, _VP, _VP, _I, _VP, _VP, _CP, _SZ]),
        "julia_hip_scratch_new": (_VP, [_SZ, _SZ, _CP, _SZ]),
        "julia_hip_scratch_free": (None, [_VP]),
        "julia_hip_gemm": (_I, [ctypes.POINTER(GemmArgs), GemmConfig, _VP, _VP, _CP, _SZ]),
        "julia_hip_gemm_static": (_I, [ctypes.POINTER(GemmArgs), GemmConfig, _VP, _CP, _SZ]),
        "julia_hip_attention": (_I, [_VP, _VP, _I, _I, _I, _I, _VP, _VP, _CP, _SZ]),
        "julia_hip_attention_seg": (_I, [_VP, _VP, _I, _I, _I, _VP, _VP, _VP, _CP, _SZ]),
        "julia_hip_embed": (_I, [_VP, _I, _VP, _I, _I, _VP, _F, _VP, _VP, _CP, _SZ]),
        "julia_hip_norm_add": (_I, [_VP, _I, _I, _VP, _VP, _F, _VP, _VP, _VP, _CP, _SZ]),
        "julia_hip_score": (_I, [_VP, _I, _I, _VP, _F, _VP, _I, _VP, _VP, _CP, _SZ]),
        "julia_hip_time_gemm": (_I, [ctypes.POINTER(GemmArgs), GemmConfig, _VP, _I, _I, _I,
                                     ctypes.POINTER(_F), ctypes.POINTER(_F), _CP, _SZ]),
        "julia_hip_time_attention": (_I, [_VP, _VP, _I, _I, _I, _I, _VP, _I, _I, _I,
                                          ctypes.POINTER(_F), ctypes.POINTER(_F), _CP, _SZ]),
        "julia_hip_time_copy": (_I, [_SZ, _I, _I, _I, ctypes.POINTER(_F), ctypes.POINTER(_F),
                                     _CP, _SZ]),
        "julia_hip_copy": (_I, [_VP, _VP, _SZ, _I, _CP, _SZ]),
        "julia_hip_device_count": (_I, []),
        "julia_hip_device_alloc": (_VP, [_SZ, _CP, _SZ]),
        "julia_hip_device_free": (None, [_VP]),
        "julia_hip_device_sync": (_I, [_CP, _SZ]),
        "julia_hip_prep_fold_layernorm": (None, [_F32P, _F32P, _I, _I, _U16P, _F32P]),
        "julia_hip_prep_fold_layernorm_bias": (None, [_F32P, _F32P, _F32P, _F32P, _I, _I, _U16P,
                                                      _F32P, _F32P]),
        "julia_hip_prep_geglu_rows": (None, [_I, _I32P]),
        "julia_hip_prep_pack_frag": (None, [_U16P, _I, _I, _U16P]),
        "julia_hip_prep_unpack_frag": (None, [_U16P, _I, _I, _U16P]),
        "julia_hip_prep_rope_table": (None, [_F, _I, _F32P]),
        "julia_hip_synth": (None, [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint64,
                                   ctypes.c_uint64, ctypes.c_double, ctypes.c_double, _F32P]),
        "julia_hip_round_f16": (None, [_F32P, _U16P, _SZ]),
        "julia_hip_answer": (_I, [ctypes.c_uint32, _F32P, _SZ, _F64P, ctypes.POINTER(ctypes.c_double),
                                  _CP, _SZ]),
        "julia_hip_latency_summary": (_I, [_F64P, _SZ, _F64P]),
        "julia_hip_gemm_choose": (GemmConfig, [_I, _I, _I, _I, _I]),
        "julia_hip_gemm_check": (_I, [ctypes.POINTER(GemmArgs), GemmConfig, _SZ, _SZ, _CP, _SZ]),
        "julia_hip_gemm_plan_2080ti": (None, [_I, _I, _I, _I, _I, ctypes.POINTER(_I),
                                              ctypes.POINTER(_I)]),
        "julia_hip_gemm_choose_2080ti": (GemmConfig, [_I, _I, _I, _I]),
        "julia_hip_engine_info_get": (_I, [_VP, ctypes.POINTER(EngineInfo)]),
        "julia_hip_checkpoint_config": (_I, [_CP, ctypes.POINTER(EngineInfo), _CP, _SZ]),
        "julia_hip_engine_tensor": (_VP, [_VP, _CP, _I, ctypes.POINTER(_SZ)]),
        "julia_hip_time_encoder_step": (_I, [_VP, _I, _I, _I, _I, _I, _I, _I, ctypes.POINTER(_F),
                                             ctypes.POINTER(_F), _CP, _SZ]),
        "julia_hip_profile_layer": (_I, [_VP, _I, _I, _VP, _VP, _I, ctypes.POINTER(_I), _VP, _CP,
                                         _SZ]),
        "julia_hip_run_trace": (_I, [_VP, _VP, _SZ, _VP, _SZ, ctypes.c_uint32, _I, _VP, _VP, _VP,
                                     _CP, _SZ]),
        "julia_hip_encode_batch": (_I, [_VP, _SZ, _VP, _VP, _I, _VP, ctypes.POINTER(_F), _CP,
                                        _SZ]),
        "julia_hip_encode_batch_phases": (_I, [_VP, _SZ, _VP, _VP, ctypes.POINTER(_F), _CP, _SZ]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _LIB = L
    return L


def _err():
    return ctypes.create_string_buffer(ERR_LEN)


def _call(fn, *args):
    e = _err()
    rc = fn(*args, e, ERR_LEN)
    if rc != 0:
        raise JuliaHipError(e.value.decode(errors="replace"))


def _np_ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _finalize(obj, _is_finalizing=sys.is_finalizing):
    """Garbage-collected objects free their device memory, except at interpreter shutdown: then
    the HIP runtime may already be torn down, so no device call is made (the process's memory
    goes with it). Callers close() what they own before exiting. (The finalizers hold this
    function and sys.is_finalizing as default arguments: at shutdown the module's globals may
    already be gone when they run.)"""
    if _is_finalizing():
        obj.ptr = None
    else:
        obj.close()


def tier():
    return lib().julia_cuda_tier().decode()


def profiler_attached(environ=None):
    """The reason a profiler is attached to this process (rocprofv3's tool library preloaded, or
    its ROCP_* / ROCPROF_* settings in the environment), or None. The measurement tools refuse
    the persistent kernel's cooperative launches under one: rocprofv3 has ended such runs with a
    segmentation fault in its own teardown, after the program's last line."""
    env = os.environ if environ is None else environ
    pre = env.get("LD_PRELOAD", "")
    if "rocprof" in pre or "roctracer" in pre:
        return "LD_PRELOAD names a profiler library (" + pre + ")"
    names = sorted(k for k in env if k.startswith(("ROCP_", "ROCPROF_")))
    if names:
        return "the environment sets " + ", ".join(names)
    return None


def refuse_cooperative_under_profiler(what):
    """Exits with a message when a profiler is attached and `what` makes cooperative launches."""
    why = profiler_attached()
    if why:
        sys.exit(f"{what} makes cooperative launches (the persistent kernel), which are not run "
                 f"under a profiler here: {why}. Time the persistent kernel with its in-kernel "
                 "stamps (profile.py) and HIP events, or profile the per-step kernels only.")


def device_count():
    return lib().julia_hip_device_count()


# ---------------------------------------------------------------- Part 1: the engine
class Engine:
    """julia_cuda_load / julia_cuda_run / julia_cuda_free (src/capi.rs)."""

    def __init__(self, spec="synthetic", max_length=0, batch_rows=0):
        """batch_rows: room for that many concatenated rows (julia_hip_load), for run_batched."""
        e = _err()
        self._free = lib().julia_cuda_free  # (held: module globals go at shutdown)
        if batch_rows:
            self.ptr = lib().julia_hip_load(spec.encode(), max_length, batch_rows, e, ERR_LEN)
        else:
            self.ptr = lib().julia_cuda_load(spec.encode(), max_length, e, ERR_LEN)
        if not self.ptr:
            raise JuliaHipError(e.value.decode(errors="replace"))

    def close(self):
        if getattr(self, "ptr", None):
            self._free(self.ptr)
            self.ptr = None

    def __del__(self, _fin=_finalize):
        _fin(self)

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def device(self):
        buf = ctypes.create_string_buffer(256)
        lib().julia_cuda_device(self.ptr, buf, 256)
        return buf.value.decode()

    def info(self):
        i = EngineInfo()
        if lib().julia_hip_engine_info_get(self.ptr, ctypes.byref(i)):
            raise JuliaHipError("no engine")
        return i

    def run(self, requests, layer_fused=False, batched=False):
        """requests: [(ids, markers, qtype)]. Returns ([logits per request], [gpu ms]).
        batched: julia_hip_run_batched (requests packed into passes over concatenated rows; a
        request's gpu ms is its pass's)."""
        ids = np.ascontiguousarray(np.concatenate([np.asarray(r[0], np.uint32) for r in requests])
                                   if requests else np.zeros(0), np.uint32)
        lens = np.array([len(r[0]) for r in requests], np.uintp)
        marks = [np.asarray(r[1], np.uint32) for r in requests]
        markers = np.ascontiguousarray(np.concatenate(marks) if marks else np.zeros(0), np.uint32)
        nm = np.array([len(m) for m in marks], np.uintp)
        qt = np.array([r[2] for r in requests], np.uint32)
        logits = np.zeros(max(len(markers), 1), np.float32)
        ms = np.zeros(max(len(requests), 1), np.float32)
        fn = lib().julia_hip_run_batched if batched else lib().julia_cuda_run
        _call(fn, self.ptr, len(requests), _np_ptr(ids), _np_ptr(lens),
              _np_ptr(markers), _np_ptr(nm), _np_ptr(qt), int(bool(layer_fused)),
              _np_ptr(logits), _np_ptr(ms))
        out, at = [], 0
        for m in nm:
            out.append(logits[at:at + m].copy())
            at += m
        return out, ms[: len(requests)].copy()

    def model_kernel(self, rows):
        """Whether layer_fused runs `rows` rows as one whole-model launch."""
        return bool(lib().julia_hip_model_kernel(self.ptr, rows))

    def run_trace(self, ids, markers, qtype, layer_fused=False, trace=True, head_x=False):
        inf = self.info()
        ids = np.ascontiguousarray(ids, np.uint32)
        markers = np.ascontiguousarray(markers, np.uint32)
        n = len(ids)
        logits = np.zeros(max(len(markers), 1), np.float32)
        xt = np.zeros((inf.layers, n, inf.d), np.uint16) if trace else None
        hx = np.zeros((n, inf.d), np.uint16) if head_x else None
        _call(lib().julia_hip_run_trace, self.ptr, _np_ptr(ids), n, _np_ptr(markers), len(markers),
              qtype, int(bool(layer_fused)), _np_ptr(logits), _np_ptr(xt), _np_ptr(hx))
        return logits[: len(markers)], xt, hx

    STEPS = {"qkv": 0, "attention": 1, "wo": 2, "wi": 3, "wo_mlp": 4, "attention_global": 5,
             "embed": 6, "norm_add": 7, "score": 8}

    def time_step(self, step, m, bm=0, splits=1, warmup=20, batches=10, per_batch=44):
        """One encoder step on m rows, rotating through the layers' weights; (min, median) us."""
        mn, md = ctypes.c_float(), ctypes.c_float()
        _call(lib().julia_hip_time_encoder_step, self.ptr, self.STEPS.get(step, step), m, bm,
              splits, warmup, batches, per_batch, ctypes.byref(mn), ctypes.byref(md))
        return mn.value, md.value

    def encode_batch(self, seqs, layer_fused=False, want_x=True):
        """Config 5's batched encoder: the id sequences concatenated, positions restarting per
        sequence, attention within each. Returns (x after the encoder [rows][d] f16 bits or None,
        GPU ms)."""
        ids = np.ascontiguousarray(np.concatenate([np.asarray(s, np.uint32) for s in seqs]),
                                   np.uint32)
        lens = np.array([len(s) for s in seqs], np.uintp)
        x = np.empty((len(ids), self.info().d), np.uint16) if want_x else None
        ms = ctypes.c_float()
        _call(lib().julia_hip_encode_batch, self.ptr, len(seqs), _np_ptr(ids), _np_ptr(lens),
              int(layer_fused), _np_ptr(x), ctypes.byref(ms))
        return x, ms.value

    def encode_batch_phases(self, seqs):
        """The batched encoder through the per-step kernels with events between the steps:
        {step: GPU ms summed over the layers}."""
        ids = np.ascontiguousarray(np.concatenate([np.asarray(s, np.uint32) for s in seqs]),
                                   np.uint32)
        lens = np.array([len(s) for s in seqs], np.uintp)
        out = (ctypes.c_float * 5)()
        _call(lib().julia_hip_encode_batch_phases, self.ptr, len(seqs), _np_ptr(ids),
              _np_ptr(lens), out)
        return dict(zip(("qkv", "attention", "wo", "wi", "wo_mlp"), [float(v) for v in out]))

    def profile_layer(self, n, layer=1, plan=None):
        """The persistent encoder kernel's per-block phase stamps (src/profile.rs): returns (plan,
        stamps [grid][layers][PROF_WORDS] u64 of a 100 MHz clock). layer -1: the whole encoder in one
        launch, as the forward pass runs it; otherwise that one layer."""
        layers = self.info().layers if layer < 0 else 1
        rows = 1024 * layers
        stamps = np.zeros((rows, PROF_WORDS), np.uint64)
        grid = ctypes.c_int()
        pin = None if plan is None else np.ascontiguousarray(plan, np.int32)
        pout = np.zeros(10, np.int32)
        _call(lib().julia_hip_profile_layer, self.ptr, n, layer, _np_ptr(pin), _np_ptr(stamps),
              rows, ctypes.byref(grid), _np_ptr(pout))
        return pout, stamps[: grid.value * layers].reshape(grid.value, layers, PROF_WORDS)

    def tensor(self, name, index=0):
        """(device address, bytes) of a prepared weight tensor."""
        nb = ctypes.c_size_t()
        p = lib().julia_hip_engine_tensor(self.ptr, name.encode(), index, ctypes.byref(nb))
        if not p:
            raise KeyError(f"{name}[{index}]")
        return p, nb.value

    def tensor_host(self, name, index=0, dtype=np.uint16):
        p, nb = self.tensor(name, index)
        out = np.empty(nb // np.dtype(dtype).itemsize, dtype)
        copy(_np_ptr(out).value, p, nb, kind=2)
        return out


def checkpoint_config(path):
    """The model config a checkpoint directory implies (checked, without a GPU)."""
    i = EngineInfo()
    _call(lib().julia_hip_checkpoint_config, path.encode(), ctypes.byref(i))
    return i


def copy(dst, src, nbytes, kind=4):
    """hipMemcpy: kind 1 host->device, 2 device->host, 3 device->device, 4 default."""
    _call(lib().julia_hip_copy, dst, src, nbytes, kind)


def sync():
    _call(lib().julia_hip_device_sync)


class DeviceBuffer:
    """Device memory from this library's own HIP runtime (julia_hip_device_alloc): for callers
    that do not bring a HIP binding (bench.py). `ptr` is the device address."""

    def __init__(self, nbytes):
        e = _err()
        self._free = lib().julia_hip_device_free  # (held: module globals go at shutdown)
        self.nbytes = int(nbytes)
        self.ptr = lib().julia_hip_device_alloc(self.nbytes, e, ERR_LEN)
        if not self.ptr:
            raise JuliaHipError(e.value.decode(errors="replace"))

    @classmethod
    def of(cls, a):
        """A buffer holding a copy of the numpy array a."""
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        copy(b.ptr, _np_ptr(a).value, a.nbytes, kind=1)
        return b

    def to_host(self, dtype, shape):
        out = np.empty(shape, dtype)
        copy(_np_ptr(out).value, self.ptr, out.nbytes, kind=2)
        return out

    def close(self):
        if getattr(self, "ptr", None):
            self._free(self.ptr)
            self.ptr = None

    def __del__(self, _fin=_finalize):
        _fin(self)


# ---------------------------------------------------------------- Part 2: per-op surface
class Scratch:
    """Split-K / key-range partials and arrival counters (src/gemm.rs `Scratch`)."""

    def __init__(self, ws_floats=1 << 22, counters=1 << 16):
        e = _err()
        self._free = lib().julia_hip_scratch_free  # (held: module globals go at shutdown)
        self.ptr = lib().julia_hip_scratch_new(ws_floats, counters, e, ERR_LEN)
        if not self.ptr:
            raise JuliaHipError(e.value.decode(errors="replace"))

    def close(self):
        if getattr(self, "ptr", None):
            self._free(self.ptr)
            self.ptr = None

    def __del__(self, _fin=_finalize):
        _fin(self)


def gemm_args(epi, a, w, c, m, n, k, stats_in=0, colsum=0, eps=1e-5, bias=0, rope=0, positions=0,
              rope_rows=0, stats_out=0):
    if isinstance(epi, str):
        epi = EPI[epi]
    return GemmArgs(epi, a, w, c, m, n, k, stats_in or None, colsum or None, eps, bias or None,
                    rope or None, positions or None, rope_rows, stats_out or None)


def gemm(args, bm=0, splits=1, scratch=None, stream=0):
    _call(lib().julia_hip_gemm, ctypes.byref(args), GemmConfig(bm, splits),
          scratch.ptr if scratch else None, stream or None)


def gemm_static(args, bm=0, splits=1, stream=0):
    """julia_hip_gemm without a scratch argument: the library's static device scratch."""
    _call(lib().julia_hip_gemm_static, ctypes.byref(args), GemmConfig(bm, splits), stream or None)


def time_gemm(args, bm=0, splits=1, scratch=None, warmup=20, batches=10, per_batch=50):
    mn, md = ctypes.c_float(), ctypes.c_float()
    _call(lib().julia_hip_time_gemm, ctypes.byref(args), GemmConfig(bm, splits),
          scratch.ptr if scratch else None, warmup, batches, per_batch, ctypes.byref(mn),
          ctypes.byref(md))
    return mn.value, md.value


def attention(qkv, o, n, d, window=0, chunks=1, scratch=None, stream=0):
    _call(lib().julia_hip_attention, qkv, o, n, d, window, chunks,
          scratch.ptr if scratch else None, stream or None)


def attention_seg(qkv, o, n, d, window, seg, scratch=None, stream=0):
    """Attention over concatenated sequences: seg is the device address of [n][2] int32 bounds."""
    _call(lib().julia_hip_attention_seg, qkv, o, n, d, window, seg,
          scratch.ptr if scratch else None, stream or None)


def time_attention(qkv, o, n, d, window=0, chunks=1, scratch=None, warmup=20, batches=10,
                   per_batch=50):
    mn, md = ctypes.c_float(), ctypes.c_float()
    _call(lib().julia_hip_time_attention, qkv, o, n, d, window, chunks,
          scratch.ptr if scratch else None, warmup, batches, per_batch, ctypes.byref(mn),
          ctypes.byref(md))
    return mn.value, md.value


def time_copy(nbytes, warmup=20, batches=10, per_batch=50):
    """(min, median) microseconds of the library's plain device copy of nbytes."""
    mn, md = ctypes.c_float(), ctypes.c_float()
    _call(lib().julia_hip_time_copy, nbytes, warmup, batches, per_batch, ctypes.byref(mn),
          ctypes.byref(md))
    return mn.value, md.value


def embed(ids, n, table, vocab, d, gamma, eps, x, stream=0):
    _call(lib().julia_hip_embed, ids, n, table, vocab, d, gamma, eps, x, stream or None)


def norm_add(x, n, d, gamma, add, eps, out, stats, stream=0):
    _call(lib().julia_hip_norm_add, x, n, d, gamma, add, eps, out, stats, stream or None)


def score(y, n, d, w, b, markers, k, logits, stream=0):
    _call(lib().julia_hip_score, y, n, d, w, b, markers, k, logits, stream or None)


# ---------------------------------------------------------------- Part 3: host logic
def fold_layernorm(w, gamma):
    w = np.ascontiguousarray(w, np.float32)
    out, k = w.shape
    w16 = np.empty((out, k), np.uint16)
    cs = np.empty(out, np.float32)
    lib().julia_hip_prep_fold_layernorm(w, np.ascontiguousarray(gamma, np.float32), out, k, w16, cs)
    return w16, cs


def fold_layernorm_bias(w, gamma, beta, b):
    w = np.ascontiguousarray(w, np.float32)
    out, k = w.shape
    w16 = np.empty((out, k), np.uint16)
    cs = np.empty(out, np.float32)
    bias = np.empty(out, np.float32)
    f32 = lambda v: np.ascontiguousarray(v, np.float32)
    lib().julia_hip_prep_fold_layernorm_bias(w, f32(gamma), f32(beta), f32(b), out, k, w16, cs, bias)
    return w16, cs, bias


def geglu_rows(inter):
    src = np.empty(2 * inter, np.int32)
    lib().julia_hip_prep_geglu_rows(inter, src)
    return src


def pack_frag(w16):
    """w16 [n][k] f16 bits -> the GEMM kernels' MFMA fragment order (a flat array)."""
    w16 = np.ascontiguousarray(w16, np.uint16)
    n, k = w16.shape
    if n % 64 or k % 32:
        raise JuliaHipError(f"pack_frag: {n} x {k} is not a multiple of 64 x 32")
    out = np.empty(n * k, np.uint16)
    lib().julia_hip_prep_pack_frag(w16, n, k, out)
    return out


def unpack_frag(packed, n, k):
    if n % 64 or k % 32 or packed.size != n * k:
        raise JuliaHipError(f"unpack_frag: {packed.size} values for {n} x {k}")
    w = np.empty((n, k), np.uint16)
    lib().julia_hip_prep_unpack_frag(np.ascontiguousarray(packed, np.uint16).ravel(), n, k, w)
    return w


def rope_table(theta, npos):
    t = np.empty((npos, 32, 2), np.float32)
    lib().julia_hip_prep_rope_table(theta, npos, t)
    return t


def synth(seed, tid, count, mean, std, start=0):
    out = np.empty(count, np.float32)
    lib().julia_hip_synth(seed, tid, start, count, mean, std, out)
    return out


def round_f16(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().julia_hip_round_f16(x.ravel(), out.ravel(), x.size)
    return out


def gemm_choose(m, n, k, cus=256, epi=0):
    if isinstance(epi, str):
        epi = EPI[epi]
    c = lib().julia_hip_gemm_choose(m, n, k, cus, epi)
    return c.bm, c.splits


def gemm_check(args, bm, splits=1, ws_floats=0, counters=0):
    """The launcher's precondition checks on the host (no device): raises JuliaHipError."""
    _call(lib().julia_hip_gemm_check, ctypes.byref(args), GemmConfig(bm, splits), ws_floats,
          counters)


def gemm_plan_2080ti(n, cols, k, sms=68, per_sm=2):
    bm, sp = ctypes.c_int(), ctypes.c_int()
    lib().julia_hip_gemm_plan_2080ti(n, cols, k, sms, per_sm, ctypes.byref(bm), ctypes.byref(sp))
    return bm.value, sp.value


def gemm_choose_2080ti(m, n, k, sms=68):
    c = lib().julia_hip_gemm_choose_2080ti(m, n, k, sms)
    return c.bm, c.splits


QTYPES = ("choice", "score", "noul")
SERVE_PATH = os.path.join(_HERE, "lib", "julia-serve")


def answer(qtype, logits):
    """julia-rs head::answer (julia_hip_answer): (value, probabilities); value is the chosen
    index (choice), the expected index (score) or p[1] (noul)."""
    if isinstance(qtype, str):
        qtype = QTYPES.index(qtype)
    lg = np.ascontiguousarray(logits, np.float32)
    p = np.zeros(max(len(lg), 1), np.float64)
    v = ctypes.c_double()
    _call(lib().julia_hip_answer, qtype, lg, len(lg), p, ctypes.byref(v))
    return (int(v.value) if qtype == 0 else v.value), p[: len(lg)]


def latency_summary(values):
    """src/serve.rs:78-115 report's (mean, p50, p90, p99, max)."""
    v = np.ascontiguousarray(values, np.float64)
    out = np.zeros(5, np.float64)
    if lib().julia_hip_latency_summary(v, len(v), out):
        raise JuliaHipError("latency_summary: no values")
    return tuple(float(x) for x in out)
