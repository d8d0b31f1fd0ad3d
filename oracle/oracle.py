"""ctypes binding of the CPU checker -- TEST INFRASTRUCTURE ONLY.

Loads oracle/liborc_sampler.so (the restatement of the reference sampler,
sampler_oracle.cpp) and, when it was built, oracle/_ref/libref_sampler.so (the
reference's own src/sampler/sampler.cpp behind a C ABI, ref_wrap.cpp). Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "liborc_sampler.so"
REF_SO = HERE / "_ref" / "libref_sampler.so"

PARAM_FIELDS = (
    "rep_penalty", "repeat_last_n", "dry_multiplier", "dry_base", "dry_allowed_len",
    "dry_last_n", "frequency_penalty", "presence_penalty", "temperature", "top_k",
    "top_p", "min_p",
)


class OrcParams(ctypes.Structure):
    _fields_ = [
        ("rep_penalty", ctypes.c_float),
        ("repeat_last_n", ctypes.c_uint64),
        ("dry_multiplier", ctypes.c_float),
        ("dry_base", ctypes.c_float),
        ("dry_allowed_len", ctypes.c_uint64),
        ("dry_last_n", ctypes.c_uint64),
        ("frequency_penalty", ctypes.c_float),
        ("presence_penalty", ctypes.c_float),
        ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_uint64),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
    ]


class OrcTrace(ctypes.Structure):
    _fields_ = [
        ("cap", ctypes.c_int32),
        ("topk_count", ctypes.c_int32),
        ("topk_idx", ctypes.POINTER(ctypes.c_int32)),
        ("kept_count", ctypes.c_int32),
        ("kept_idx", ctypes.POINTER(ctypes.c_int32)),
        ("kept_prob", ctypes.POINTER(ctypes.c_float)),
        ("u_consumed", ctypes.c_int32),
        ("greedy", ctypes.c_int32),
        ("cdf_margin", ctypes.c_double),
        ("topp_margin", ctypes.c_double),
    ]


def identity_params(**over) -> dict:
    """SamplerParams::identity() (reference src/sampler/sampler.cpp:192-205)."""
    p = dict(rep_penalty=1.0, repeat_last_n=0, dry_multiplier=0.0, dry_base=1.75,
             dry_allowed_len=2, dry_last_n=0, frequency_penalty=0.0, presence_penalty=0.0,
             temperature=1.0, top_k=0, top_p=1.0, min_p=0.0)
    p.update(over)
    return p


def default_params(**over) -> dict:
    """SamplerParams{} (reference include/ultima/sampler/sampler.hpp:16-52)."""
    p = dict(rep_penalty=1.1, repeat_last_n=64, dry_multiplier=0.8, dry_base=1.75,
             dry_allowed_len=2, dry_last_n=512, frequency_penalty=0.0, presence_penalty=0.0,
             temperature=0.2, top_k=40, top_p=0.95, min_p=0.05)
    p.update(over)
    return p


def to_orc(p: dict) -> OrcParams:
    o = OrcParams()
    for k in PARAM_FIELDS:
        setattr(o, k, p[k])
    return o


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not ORACLE_SO.exists():
            raise RuntimeError(f"{ORACLE_SO} is not built (run __graft_entry__.build())")
        L = ctypes.CDLL(str(ORACLE_SO))
        i32, i64, u64, f32, f64 = (ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64,
                                   ctypes.c_float, ctypes.c_double)
        vp = ctypes.c_void_p
        L.orc_sample_row.restype = i32
        L.orc_sample_row.argtypes = [vp, i64, ctypes.POINTER(OrcParams), vp, i64, vp, vp, vp,
                                     i64, f64, ctypes.POINTER(OrcTrace)]
        L.orc_argmax.restype = i32
        L.orc_argmax.argtypes = [vp, i64]
        L.orc_sample_batch.restype = None
        L.orc_sample_batch.argtypes = [vp, i64, i64, i64, vp, vp, i64, vp, vp, i64, vp, vp, i32]
        L.orc_sample_batch_stages.restype = None
        L.orc_sample_batch_stages.argtypes = [vp, i64, i64, i64, vp, vp, i64, vp, vp, i64, vp, vp, vp]
        L.orc_u_from_seed.restype = f64
        L.orc_u_from_seed.argtypes = [u64]
        L.orc_mt19937_64_nth.restype = u64
        L.orc_mt19937_64_nth.argtypes = [u64, u64]
        L.orc_expf.restype = f32
        L.orc_expf.argtypes = [f32]
        L.orc_powf.restype = f32
        L.orc_powf.argtypes = [f32, f32]
        L.orc_expf_many.restype = None
        L.orc_expf_many.argtypes = [vp, vp, i64, i32]
        _lib = L
    return _lib


def ref_available() -> bool:
    return REF_SO.exists()


def ref():
    global _ref
    if _ref is None:
        if not REF_SO.exists():
            raise RuntimeError(f"{REF_SO} is not built (reference sources absent?)")
        R = ctypes.CDLL(str(REF_SO))
        vp, i32, i64, u64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64
        R.ref_sample_row.restype = i32
        R.ref_sample_row.argtypes = [vp, i64, ctypes.POINTER(OrcParams), vp, i64, vp, vp, i64, u64]
        R.ref_argmax.restype = i32
        R.ref_argmax.argtypes = [vp, i64]
        R.ref_sample_batch.restype = None
        R.ref_sample_batch.argtypes = [vp, i64, i64, i64, vp, vp, i64, vp, vp, vp, i32]
        _ref = R
    return _ref


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


@dataclass
class Trace:
    token: int
    topk_idx: np.ndarray | None
    kept_idx: np.ndarray
    kept_prob: np.ndarray
    u_consumed: bool
    greedy: bool
    cdf_margin: float
    topp_margin: float
    logits_after: np.ndarray = field(repr=False, default=None)


def sample_row(logits, params: dict, hist=None, mask=None, bias=None, u: float = 0.5,
               cap: int | None = None) -> Trace:
    """Run the restatement on one row (a copy of `logits`, float32) and return
    the token, the sets it kept and the logits it left behind."""
    L = lib()
    x = np.array(logits, dtype=np.float32, copy=True)
    V = x.shape[0]
    h = None if hist is None else np.ascontiguousarray(hist, dtype=np.int32)
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint32)
    if bias:
        bid = np.array(list(bias.keys()), dtype=np.int32)
        bval = np.array(list(bias.values()), dtype=np.float32)
    else:
        bid = bval = None
    cap = V if cap is None else cap
    topk = np.zeros(max(cap, 1), np.int32)
    kidx = np.zeros(max(cap, 1), np.int32)
    kprob = np.zeros(max(cap, 1), np.float32)
    tr = OrcTrace(cap=cap, topk_idx=topk.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                  kept_idx=kidx.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                  kept_prob=kprob.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    op = to_orc(params)
    tok = L.orc_sample_row(_ptr(x), V, ctypes.byref(op), _ptr(h), 0 if h is None else h.shape[0],
                           _ptr(m), _ptr(bid), _ptr(bval), 0 if bid is None else bid.shape[0],
                           float(u), ctypes.byref(tr))
    tk = None if tr.topk_count < 0 else topk[:min(tr.topk_count, cap)].copy()
    n = min(tr.kept_count, cap)
    return Trace(token=int(tok), topk_idx=tk, kept_idx=kidx[:n].copy(), kept_prob=kprob[:n].copy(),
                 u_consumed=bool(tr.u_consumed), greedy=bool(tr.greedy),
                 cdf_margin=float(tr.cdf_margin), topp_margin=float(tr.topp_margin),
                 logits_after=x)


def argmax(logits) -> int:
    x = np.ascontiguousarray(logits, dtype=np.float32)
    return int(lib().orc_argmax(_ptr(x), x.shape[0]))


def u_from_seed(seed: int) -> float:
    return float(lib().orc_u_from_seed(ctypes.c_uint64(seed & (2**64 - 1))))


def mt19937_64_nth(seed: int, n: int) -> int:
    return int(lib().orc_mt19937_64_nth(seed, n))


def expf(x: float) -> float:
    return float(lib().orc_expf(x))


def powf(x: float, y: float) -> float:
    return float(lib().orc_powf(x, y))


def expf_many(x: np.ndarray, nthreads: int | None = None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    nt = nthreads or min(16, os.cpu_count() or 1)
    lib().orc_expf_many(_ptr(x), _ptr(out), x.size, nt)
    return out


def params_array(plist) -> ctypes.Array:
    arr = (OrcParams * len(plist))()
    for i, p in enumerate(plist):
        arr[i] = to_orc(p)
    return arr


def sample_batch(logits_f32: np.ndarray, plist, hist=None, hist_len=None, mask=None, u=None,
                 nthreads: int = 1) -> np.ndarray:
    """The restatement over a [B, V] float32 batch (mutated in place), rows
    split over nthreads threads. Returns the tokens."""
    L = lib()
    B, V = logits_f32.shape
    pa = params_array(plist)
    toks = np.zeros(B, np.int32)
    hl = None if hist is None else np.ascontiguousarray(hist_len, dtype=np.int64)
    L.orc_sample_batch(_ptr(logits_f32), B, V, logits_f32.strides[0] // 4,
                       ctypes.cast(pa, ctypes.c_void_p), _ptr(hist),
                       0 if hist is None else hist.strides[0] // 4, _ptr(hl), _ptr(mask),
                       0 if mask is None else mask.strides[0] // 4,
                       _ptr(np.ascontiguousarray(u, dtype=np.float64)), _ptr(toks), nthreads)
    return toks


STAGES = ("penalties", "temperature", "top_k", "top_p", "min_p", "softmax", "draw")


def sample_batch_stages(logits_f32: np.ndarray, plist, hist=None, hist_len=None, mask=None, u=None):
    """The restatement over a [B, V] float32 batch on one thread with a clock
    around each stage. Returns (tokens, {stage: seconds summed over rows})."""
    L = lib()
    B, V = logits_f32.shape
    pa = params_array(plist)
    toks = np.zeros(B, np.int32)
    ns = np.zeros(7, np.float64)
    hl = None if hist is None else np.ascontiguousarray(hist_len, dtype=np.int64)
    L.orc_sample_batch_stages(_ptr(logits_f32), B, V, logits_f32.strides[0] // 4,
                              ctypes.cast(pa, ctypes.c_void_p), _ptr(hist),
                              0 if hist is None else hist.strides[0] // 4, _ptr(hl), _ptr(mask),
                              0 if mask is None else mask.strides[0] // 4,
                              _ptr(np.ascontiguousarray(u, dtype=np.float64)), _ptr(toks), _ptr(ns))
    return toks, {k: float(v) * 1e-9 for k, v in zip(STAGES, ns)}


def ref_sample_row(logits, params: dict, hist=None, bias=None, seed: int = 0):
    """The reference's own sample() on a copy of `logits` with a context seeded
    with `seed`. Returns (token, logits_after)."""
    R = ref()
    x = np.array(logits, dtype=np.float32, copy=True)
    h = None if hist is None else np.ascontiguousarray(hist, dtype=np.int32)
    if bias:
        bid = np.array(list(bias.keys()), dtype=np.int32)
        bval = np.array(list(bias.values()), dtype=np.float32)
    else:
        bid = bval = None
    op = to_orc(params)
    tok = R.ref_sample_row(_ptr(x), x.shape[0], ctypes.byref(op), _ptr(h),
                           0 if h is None else h.shape[0], _ptr(bid), _ptr(bval),
                           0 if bid is None else bid.shape[0], ctypes.c_uint64(seed))
    return int(tok), x


def ref_argmax(logits) -> int:
    x = np.ascontiguousarray(logits, dtype=np.float32)
    return int(ref().ref_argmax(_ptr(x), x.shape[0]))


def ref_sample_batch(logits_f32: np.ndarray, plist, hist, hist_len, seeds, nthreads: int = 1):
    R = ref()
    B, V = logits_f32.shape
    pa = params_array(plist)
    toks = np.zeros(B, np.int32)
    hl = np.ascontiguousarray(hist_len, dtype=np.int64)
    sd = np.ascontiguousarray(seeds, dtype=np.uint64)
    R.ref_sample_batch(_ptr(logits_f32), B, V, logits_f32.strides[0] // 4,
                       ctypes.cast(pa, ctypes.c_void_p), _ptr(hist), hist.strides[0] // 4, _ptr(hl),
                       _ptr(sd), _ptr(toks), nthreads)
    return toks


# ---- the logits producer (final rmsnorm + lm-head matvec) ---------------------------

HEAD_SO = HERE / "liborc_head.so"
REF_KERNELS_SO = HERE / "_ref" / "libref_kernels.so"
_head = None
_refk = None


def head_lib():
    """liborc_head.so: head_oracle.c, the restatement of the reference's AVX2
    rmsnorm and matvec order."""
    global _head
    if _head is None:
        if not HEAD_SO.exists():
            raise RuntimeError(f"{HEAD_SO} is not built (run __graft_entry__.build())")
        L = ctypes.CDLL(str(HEAD_SO))
        vp, i64, f32, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int
        L.orc_rmsnorm.restype = None
        L.orc_rmsnorm.argtypes = [vp, vp, vp, i64, f32]
        L.orc_matvec_f32.restype = None
        L.orc_matvec_f32.argtypes = [vp, vp, vp, i64, i64]
        L.orc_matvec_bf16.restype = None
        L.orc_matvec_bf16.argtypes = [vp, vp, vp, i64, i64]
        L.orc_matvec.restype = None
        L.orc_matvec.argtypes = [vp, i32, vp, vp, i64, i64]
        L.orc_hadamard_fold.restype = None
        L.orc_hadamard_fold.argtypes = [vp, vp, i64, i64, vp]
        L.orc_head_row_bytes.restype = i64
        L.orc_head_row_bytes.argtypes = [i32, i64]
        L.orc_lm_head.restype = None
        L.orc_lm_head.argtypes = [vp, i64, i64, vp, f32, vp, i32, i64, f32, vp, vp, i64, vp]
        _head = L
    return _head


def ref_kernels_available() -> bool:
    return REF_KERNELS_SO.exists()


def ref_kernels():
    """_ref/libref_kernels.so: the reference's own rmsnorm_f32, matvec_f32_f32
    and matvec_bf16_f32, compiled from its sources."""
    global _refk
    if _refk is None:
        if not REF_KERNELS_SO.exists():
            raise RuntimeError(f"{REF_KERNELS_SO} is not built (reference sources absent?)")
        R = ctypes.CDLL(str(REF_KERNELS_SO))
        vp, i64, f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float
        R.ref_rmsnorm.restype = None
        R.ref_rmsnorm.argtypes = [vp, vp, vp, i64, f32]
        R.ref_matvec_f32.restype = None
        R.ref_matvec_f32.argtypes = [vp, vp, vp, i64, i64]
        R.ref_matvec_bf16.restype = None
        R.ref_matvec_bf16.argtypes = [vp, vp, vp, i64, i64]
        R.ref_matvec_q.restype = None
        R.ref_matvec_q.argtypes = [ctypes.c_int, vp, vp, vp, i64, i64]
        R.ref_hadamard_fold.restype = None
        R.ref_hadamard_fold.argtypes = [vp, vp, i64, i64, vp]
        _refk = R
    return _refk


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def rmsnorm(x, scale, eps: float, use_ref: bool = False) -> np.ndarray:
    x, scale = _f32(x), _f32(scale)
    y = np.empty_like(x)
    (ref_kernels().ref_rmsnorm if use_ref else head_lib().orc_rmsnorm)(_ptr(x), _ptr(scale), _ptr(y), x.size, eps)
    return y


# head weight types (head_oracle.c's orc_matvec numbering)
HEAD_F32, HEAD_BF16, HEAD_Q4_K, HEAD_Q5_K, HEAD_Q6_K, HEAD_Q8_0, HEAD_Q4_1, HEAD_Q5_0, HEAD_PQ2_0 = range(9)
HEAD_NAMES = {"f32": HEAD_F32, "bf16": HEAD_BF16, "q4k": HEAD_Q4_K, "q5k": HEAD_Q5_K, "q6k": HEAD_Q6_K,
              "q8_0": HEAD_Q8_0, "q4_1": HEAD_Q4_1, "q5_0": HEAD_Q5_0, "pq2_0": HEAD_PQ2_0}


def head_row_bytes(dtype: int, H: int) -> int:
    """Bytes of one head row of H values (0 when H does not split into blocks)."""
    return int(head_lib().orc_head_row_bytes(dtype, H))


def matvec(w, x, use_ref: bool = False, dtype: int | None = None) -> np.ndarray:
    """y = W x in the reference's order; W f32 [M, K], bf16 bits (uint16) [M, K],
    or a quantised head (uint8 [M, row_bytes], `dtype` one of HEAD_Q*), K = x.size."""
    x = _f32(x)
    K = x.size
    M = w.shape[0]
    y = np.empty(M, np.float32)
    if dtype is not None and dtype >= HEAD_Q4_K:
        w = np.ascontiguousarray(w, dtype=np.uint8)
        if use_ref:
            ref_kernels().ref_matvec_q(dtype, _ptr(w), _ptr(x), _ptr(y), M, K)
        else:
            head_lib().orc_matvec(_ptr(w), dtype, _ptr(x), _ptr(y), M, K)
        return y
    if w.dtype == np.uint16:
        w = np.ascontiguousarray(w)
        fn = ref_kernels().ref_matvec_bf16 if use_ref else head_lib().orc_matvec_bf16
    else:
        w = _f32(w)
        fn = ref_kernels().ref_matvec_f32 if use_ref else head_lib().orc_matvec_f32
    fn(_ptr(w), _ptr(x), _ptr(y), M, K)
    return y


def hadamard_fold(x, block: int, signs=None, use_ref: bool = False) -> np.ndarray:
    """The reference's hadamard_fold_f32 of one row (src/kernels/hadamard.cpp:26-44)."""
    x = _f32(x)
    y = np.empty_like(x)
    sg = None if signs is None else _f32(signs)
    fn = ref_kernels().ref_hadamard_fold if use_ref else head_lib().orc_hadamard_fold
    fn(_ptr(x), _ptr(y), x.size, block, None if sg is None else _ptr(sg))
    return y


def lm_head(hidden, norm_scale, eps: float, weight, logit_scale: float = 1.0, dtype: int | None = None,
            fold_block: int = 0, fold_signs=None):
    """Logits [rows, V] of hidden states [rows, H] (reference
    src/model/qwen_model.cpp:182-207); also returns the head's input rows (the
    normed rows, folded when fold_block > 0). `dtype`: a HEAD_* type; by default
    f32 or bf16 from the weight array's element type."""
    hidden = _f32(np.atleast_2d(hidden))
    rows, H = hidden.shape
    V = weight.shape[0]
    if dtype is None:
        dtype = HEAD_BF16 if weight.dtype == np.uint16 else HEAD_F32
    if dtype == HEAD_F32:
        w = _f32(weight)
    else:
        w = np.ascontiguousarray(weight)
    sg = None if fold_signs is None else _f32(fold_signs)
    logits = np.empty((rows, V), np.float32)
    normed = np.empty((rows, H), np.float32)
    head_lib().orc_lm_head(_ptr(hidden), rows, H, _ptr(_f32(norm_scale)), eps, _ptr(w), dtype, V,
                           logit_scale, _ptr(logits), _ptr(normed), fold_block, None if sg is None else _ptr(sg))
    return logits, normed
