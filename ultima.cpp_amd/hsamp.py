"""ctypes binding of libultima_hsamp (include/ultima_hsamp.h).

PyTorch is used only to own device memory and streams; every sampling
decision is made by the library's HIP kernels. Loading fails loudly when the
library is not built.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libultima_hsamp.so"
NOALLOC_LIB_PATH = PKG / "libultima_hsamp_noalloc.so"
HEADER = PKG.parent / "include" / "ultima_hsamp.h"
NOALLOC_HEADER = PKG.parent / "include" / "ultima_hsamp_noalloc.h"

OK, ERR_INVALID, ERR_HIP, ERR_UNSUPPORTED, ERR_NOMEM, ERR_CAPACITY, ERR_NO_DEVICE = 0, -1, -2, -3, -4, -5, -6
F32, BF16 = 0, 1
WRITEBACK, STREAM_ONLY = 1, 0x100
NOALLOC_SCRATCH_BYTES, NOALLOC_PLAN_BYTES = 96 << 20, 2 << 20
KERNELS_EXACT, KERNELS_GENERAL, KERNELS_FULL, KERNELS_WRITEBACK = 1, 2, 4, 8
ROW_GREEDY, ROW_U_USED, ROW_CDF_NEAR, ROW_NAN, ROW_UNIFORM, ROW_TOPP_NEAR, ROW_REREAD = 1, 2, 4, 8, 16, 32, 64

PARAM_KEYS = ("rep_penalty", "dry_multiplier", "dry_base", "frequency_penalty", "presence_penalty",
              "temperature", "top_p", "min_p", "repeat_last_n", "dry_allowed_len", "dry_last_n",
              "top_k")


class Params(ctypes.Structure):
    _fields_ = [
        ("rep_penalty", ctypes.c_float),
        ("dry_multiplier", ctypes.c_float),
        ("dry_base", ctypes.c_float),
        ("frequency_penalty", ctypes.c_float),
        ("presence_penalty", ctypes.c_float),
        ("temperature", ctypes.c_float),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("repeat_last_n", ctypes.c_uint64),
        ("dry_allowed_len", ctypes.c_uint64),
        ("dry_last_n", ctypes.c_uint64),
        ("top_k", ctypes.c_uint64),
        ("hist_len", ctypes.c_int64),
        ("bias_offset", ctypes.c_int64),
        ("bias_count", ctypes.c_int64),
    ]


class Batch(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
        ("logits", ctypes.c_void_p),
        ("logits_stride", ctypes.c_int64),
        ("hist", ctypes.c_void_p),
        ("hist_stride", ctypes.c_int64),
        ("mask", ctypes.c_void_p),
        ("mask_stride", ctypes.c_int64),
        ("u", ctypes.c_void_p),
        ("params", ctypes.POINTER(Params)),
        ("bias_ids", ctypes.c_void_p),
        ("bias_vals", ctypes.c_void_p),
        ("token", ctypes.c_void_p),
        ("row_flags", ctypes.c_void_p),
        ("topk_idx", ctypes.c_void_p),
        ("topk_count", ctypes.c_void_p),
        ("kept_idx", ctypes.c_void_p),
        ("kept_prob", ctypes.c_void_p),
        ("kept_count", ctypes.c_void_p),
        ("set_cap", ctypes.c_int32),
        ("hist_len_dev", ctypes.c_void_p),
    ]


class Head(ctypes.Structure):
    """ultima_hsamp_head (include/ultima_hsamp.h)."""
    _fields_ = [
        ("hidden", ctypes.c_void_p),
        ("hidden_stride", ctypes.c_int64),
        ("rows", ctypes.c_int32),
        ("hidden_dim", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("weight_dtype", ctypes.c_int32),
        ("norm_scale", ctypes.c_void_p),
        ("eps", ctypes.c_float),
        ("logit_scale", ctypes.c_float),
        ("weight", ctypes.c_void_p),
        ("normed", ctypes.c_void_p),
        ("logits", ctypes.c_void_p),
        ("logits_stride", ctypes.c_int64),
        ("fold_block", ctypes.c_int32),
        ("fold_signs", ctypes.c_void_p),
    ]


class Commit(ctypes.Structure):
    """ultima_hsamp_commit (include/ultima_hsamp.h)."""
    _fields_ = [
        ("hist", ctypes.c_void_p),
        ("hist_stride", ctypes.c_int64),
        ("hist_len_dev", ctypes.c_void_p),
        ("active", ctypes.c_void_p),
        ("budget", ctypes.c_void_p),
        ("keep", ctypes.c_int32),
        ("n_stop", ctypes.c_int32),
        ("stop_ids", ctypes.c_void_p),
    ]


class Verify(ctypes.Structure):
    """ultima_hsamp_verify (include/ultima_hsamp.h)."""
    _fields_ = [
        ("n_pos", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("logits", ctypes.c_void_p),
        ("logits_stride", ctypes.c_int64),
        ("draft", ctypes.c_void_p),
        ("hist", ctypes.c_void_p),
        ("hist_len", ctypes.c_int32),
        ("mask", ctypes.c_void_p),
        ("mask_stride", ctypes.c_int64),
        ("u", ctypes.c_void_p),
        ("params", ctypes.POINTER(Params)),
        ("bias_ids", ctypes.c_void_p),
        ("bias_vals", ctypes.c_void_p),
        ("work", ctypes.c_void_p),
        ("out_tokens", ctypes.c_void_p),
        ("out_count", ctypes.c_void_p),
        ("row_flags", ctypes.c_void_p),
    ]


def declared_symbols(header: Path = HEADER) -> list[str]:
    """Function names declared in a header (default include/ultima_hsamp.h)."""
    import re
    text = header.read_text()
    return sorted(set(re.findall(r"\b(ultima_hsamp_[a-z_0-9]+)\s*\(", text)))


_lib = None


def lib() -> ctypes.CDLL:
    """Load libultima_hsamp.so. PyTorch-ROCm ships its own HIP runtime with the
    same SONAME as ROCm's; importing torch first makes the library bind to that
    one instance, since one process cannot hold two HSA runtimes."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build()")
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i32, i64, f64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_double
        L.ultima_hsamp_create.restype = ctypes.c_int
        L.ultima_hsamp_create.argtypes = [ctypes.c_int, i32, i32, ctypes.POINTER(vp)]
        L.ultima_hsamp_destroy.restype = ctypes.c_int
        L.ultima_hsamp_destroy.argtypes = [vp]
        L.ultima_hsamp_run.restype = ctypes.c_int
        L.ultima_hsamp_run.argtypes = [vp, ctypes.POINTER(Batch), vp]
        L.ultima_hsamp_sample_host.restype = ctypes.c_int
        L.ultima_hsamp_sample_host.argtypes = [vp, vp, i32, ctypes.POINTER(Params), vp, vp, vp, f64,
                                               ctypes.c_int, ctypes.POINTER(i32)]
        L.ultima_hsamp_params_default.restype = None
        L.ultima_hsamp_params_default.argtypes = [ctypes.POINTER(Params)]
        L.ultima_hsamp_params_identity.restype = None
        L.ultima_hsamp_params_identity.argtypes = [ctypes.POINTER(Params)]
        L.ultima_hsamp_uniform_from_u64.restype = f64
        L.ultima_hsamp_uniform_from_u64.argtypes = [ctypes.c_uint64]
        L.ultima_hsamp_status_str.restype = ctypes.c_char_p
        L.ultima_hsamp_status_str.argtypes = [ctypes.c_int]
        L.ultima_hsamp_version.restype = ctypes.c_int
        L.ultima_hsamp_version.argtypes = []
        L.ultima_hsamp_query_kernels.restype = ctypes.c_int
        L.ultima_hsamp_query_kernels.argtypes = [vp, ctypes.POINTER(Batch), ctypes.POINTER(ctypes.c_uint32)]
        L.ultima_hsamp_read_probe.restype = ctypes.c_int
        L.ultima_hsamp_read_probe.argtypes = [vp, ctypes.POINTER(Batch), vp, vp]
        L.ultima_hsamp_set_phase_event.restype = ctypes.c_int
        L.ultima_hsamp_set_phase_event.argtypes = [vp, vp]
        L.ultima_hsamp_history_push.restype = ctypes.c_int
        L.ultima_hsamp_history_push.argtypes = [vp, ctypes.c_int64, vp, vp, i32, i32, vp]
        L.ultima_hsamp_lm_head.restype = ctypes.c_int
        L.ultima_hsamp_lm_head.argtypes = [ctypes.POINTER(Head), vp]
        L.ultima_hsamp_decode_commit.restype = ctypes.c_int
        L.ultima_hsamp_decode_commit.argtypes = [vp, i64, vp, vp, vp, vp, i32, i32, vp, i32, vp]
        L.ultima_hsamp_run_commit.restype = ctypes.c_int
        L.ultima_hsamp_run_commit.argtypes = [vp, ctypes.POINTER(Batch), ctypes.POINTER(Commit), vp]
        L.ultima_hsamp_verify_work_ints.restype = i64
        L.ultima_hsamp_verify_work_ints.argtypes = [i32, i32]
        L.ultima_hsamp_verify_block.restype = ctypes.c_int
        L.ultima_hsamp_verify_block.argtypes = [vp, ctypes.POINTER(Verify), vp]
        _lib = L
    return _lib


class HsampError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what}: {status} ({lib().ultima_hsamp_status_str(status).decode()})")


def check(status: int, what: str) -> None:
    if status != OK:
        raise HsampError(status, what)


def make_params(plist, hist_len=None, bias=None):
    """(ctypes array of Params, bias ids array, bias values array) for a list of
    knob dicts. bias: list (per row) of {id: value} or None."""
    B = len(plist)
    arr = (Params * B)()
    ids, vals = [], []
    for r, p in enumerate(plist):
        q = arr[r]
        for k in PARAM_KEYS:
            setattr(q, k, p[k])
        q.hist_len = 0 if hist_len is None else int(hist_len[r])
        q.bias_offset = len(ids)
        b = bias[r] if bias is not None else None
        q.bias_count = 0 if not b else len(b)
        if b:
            for t, v in b.items():
                ids.append(int(t))
                vals.append(float(v))
    bids = np.array(ids, np.int32) if ids else None
    bvals = np.array(vals, np.float32) if vals else None
    return arr, bids, bvals


def _batch(logits, params, u, hist, hist_len, mask, bias, writeback, want_sets, set_cap, stream, outputs,
           stream_only, hist_len_dev=None):
    """An ultima_hsamp_batch over torch tensors: (batch, outputs, host arrays
    the call reads, stream)."""
    import torch
    B, V = logits.shape[0], logits.shape[1]
    dev = logits.device
    out = outputs if outputs is not None else {}
    if "token" not in out:
        out["token"] = torch.empty(B, dtype=torch.int32, device=dev)
    if "row_flags" not in out:
        out["row_flags"] = torch.empty(B, dtype=torch.int32, device=dev)
    cap = 0
    if want_sets:
        cap = set_cap or V
        for k, dt in (("topk_idx", torch.int32), ("kept_idx", torch.int32),
                      ("kept_prob", torch.float32)):
            if k not in out:
                out[k] = torch.empty((B, cap), dtype=dt, device=dev)
        for k in ("topk_count", "kept_count"):
            if k not in out:
                out[k] = torch.empty(B, dtype=torch.int32, device=dev)
    parr, bids, bvals = make_params(params, hist_len, bias)
    b = Batch()
    b.rows, b.vocab = B, V
    b.dtype = F32 if logits.dtype == torch.float32 else BF16
    b.flags = (WRITEBACK if writeback else 0) | (STREAM_ONLY if stream_only else 0)
    b.logits = logits.data_ptr()
    b.logits_stride = logits.stride(0)
    if hist is not None:
        b.hist = hist.data_ptr()
        b.hist_stride = hist.stride(0)
    if hist_len_dev is not None:
        b.hist_len_dev = hist_len_dev.data_ptr()
    if mask is not None:
        b.mask = mask.data_ptr()
        b.mask_stride = mask.stride(0)
    b.u = u.data_ptr()
    b.params = ctypes.cast(parr, ctypes.POINTER(Params))
    if bids is not None:
        b.bias_ids = bids.ctypes.data
        b.bias_vals = bvals.ctypes.data
    b.token = out["token"].data_ptr()
    b.row_flags = out["row_flags"].data_ptr()
    if want_sets:
        b.topk_idx = out["topk_idx"].data_ptr()
        b.topk_count = out["topk_count"].data_ptr()
        b.kept_idx = out["kept_idx"].data_ptr()
        b.kept_prob = out["kept_prob"].data_ptr()
        b.kept_count = out["kept_count"].data_ptr()
        b.set_cap = cap
    elif "kept_count" in out:
        b.kept_count = out["kept_count"].data_ptr()   # the count alone
    s = torch.cuda.current_stream(dev) if stream is None else stream
    return b, out, (parr, bids, bvals), s


_noalloc_lib = None


def noalloc_lib() -> ctypes.CDLL:
    """Load libultima_hsamp_noalloc.so (include/ultima_hsamp_noalloc.h); it
    links libultima_hsamp.so, loaded first."""
    global _noalloc_lib
    if _noalloc_lib is None:
        lib()
        if not NOALLOC_LIB_PATH.exists():
            raise RuntimeError(f"{NOALLOC_LIB_PATH} is not built: run __graft_entry__.build()")
        L = ctypes.CDLL(str(NOALLOC_LIB_PATH))
        L.ultima_hsamp_run_noalloc.restype = ctypes.c_int
        L.ultima_hsamp_run_noalloc.argtypes = [ctypes.POINTER(Batch), ctypes.c_void_p]
        _noalloc_lib = L
    return _noalloc_lib


def run_noalloc(logits, params, u, hist=None, hist_len=None, mask=None, bias=None, writeback=False,
                want_sets=False, set_cap=None, stream=None, outputs=None):
    """ultima_hsamp_run_noalloc on the current device: Sampler.run without a
    handle, scratch from the library's fixed device array."""
    b, out, keep, s = _batch(logits, params, u, hist, hist_len, mask, bias, writeback, want_sets, set_cap,
                             stream, outputs, False)
    check(noalloc_lib().ultima_hsamp_run_noalloc(ctypes.byref(b), ctypes.c_void_p(s.cuda_stream)), "run_noalloc")
    del keep
    return out


def history_push(hist, hist_len_dev, tokens, keep: int, stream=None) -> None:
    """ultima_hsamp_history_push on torch tensors of one device: hist int32
    [rows, stride] (the rows' histories), hist_len_dev int32 [rows] (their
    lengths, advanced here), tokens int32 [rows] (appended; e.g. the token
    output of run()). A full row first keeps its last `keep` ids."""
    import torch
    rows = hist.shape[0]
    assert hist.dtype == torch.int32 and hist_len_dev.dtype == torch.int32 and tokens.dtype == torch.int32
    assert hist_len_dev.shape[0] >= rows and tokens.shape[0] >= rows and hist.stride(1) == 1
    s = torch.cuda.current_stream(hist.device) if stream is None else stream
    check(lib().ultima_hsamp_history_push(ctypes.c_void_p(hist.data_ptr()), hist.stride(0),
                                          ctypes.c_void_p(hist_len_dev.data_ptr()),
                                          ctypes.c_void_p(tokens.data_ptr()), rows, int(keep),
                                          ctypes.c_void_p(s.cuda_stream)), "history_push")


def decode_commit(hist, hist_len_dev, tokens, active, keep: int, stop_ids=(), budget=None, stream=None) -> None:
    """ultima_hsamp_decode_commit on torch tensors of one device (int32): after
    a run() over the slots' rows, ends the rows whose token is a stop id (or
    -1), marks the tokens of ended rows -1, appends the rest to the histories
    and counts them against budget (the server loop's max_tokens)."""
    import torch
    rows = hist.shape[0]
    for t in (hist, hist_len_dev, tokens, active) + ((budget,) if budget is not None else ()):
        assert t.dtype == torch.int32 and t.device == hist.device
    assert hist_len_dev.shape[0] >= rows and tokens.shape[0] >= rows and active.shape[0] >= rows
    assert hist.stride(1) == 1 and (budget is None or budget.shape[0] >= rows)
    stop = np.asarray(list(stop_ids), np.int32)
    s = torch.cuda.current_stream(hist.device) if stream is None else stream
    check(lib().ultima_hsamp_decode_commit(
        ctypes.c_void_p(hist.data_ptr()), hist.stride(0), ctypes.c_void_p(hist_len_dev.data_ptr()),
        ctypes.c_void_p(tokens.data_ptr()), ctypes.c_void_p(active.data_ptr()),
        ctypes.c_void_p(budget.data_ptr() if budget is not None else 0), rows, int(keep),
        stop.ctypes.data_as(ctypes.c_void_p) if stop.size else None, int(stop.size),
        ctypes.c_void_p(s.cuda_stream)), "decode_commit")


# head weight types (ULTIMA_HSAMP_F32 / _BF16 / _HEAD_*)
HEAD_Q4_K, HEAD_Q5_K, HEAD_Q6_K, HEAD_Q8_0, HEAD_Q4_1, HEAD_Q5_0, HEAD_PQ2_0 = range(2, 9)


def lm_head(hidden, norm_scale, eps: float, weight, logit_scale: float = 1.0, logits=None, normed=None,
            stream=None, weight_dtype=None, fold_block: int = 0, fold_signs=None):
    """ultima_hsamp_lm_head on torch tensors of one device: hidden [rows, H] f32,
    norm_scale [H] f32, weight [V, H] f32 or bf16, or a quantised head [V, row
    bytes] uint8 with weight_dtype one of HEAD_Q*; fold_block / fold_signs [H]
    f32 the Hadamard fold. Returns (logits [rows, V], normed [rows, H]); the
    outputs may be passed in (allocated otherwise)."""
    import torch
    if hidden.dim() == 1:
        hidden = hidden.unsqueeze(0)
    rows, H = hidden.shape
    V = weight.shape[0]
    dev = hidden.device
    if weight_dtype is None:
        if weight.dtype not in (torch.float32, torch.bfloat16):
            raise HsampError(ERR_INVALID, "lm_head: weight must be float32 or bfloat16 (or give weight_dtype)")
        weight_dtype = BF16 if weight.dtype == torch.bfloat16 else F32
    if logits is None:
        logits = torch.empty((rows, V), dtype=torch.float32, device=dev)
    if normed is None:
        normed = torch.empty((rows, H), dtype=torch.float32, device=dev)
    h = Head()
    h.hidden = hidden.data_ptr()
    h.hidden_stride = hidden.stride(0)
    h.rows, h.hidden_dim, h.vocab = rows, H, V
    h.weight_dtype = weight_dtype
    h.norm_scale = norm_scale.data_ptr()
    h.eps = eps
    h.logit_scale = logit_scale
    h.weight = weight.data_ptr()
    h.normed = normed.data_ptr()
    h.logits = logits.data_ptr()
    h.logits_stride = logits.stride(0)
    h.fold_block = fold_block
    h.fold_signs = None if fold_signs is None else fold_signs.data_ptr()
    s = torch.cuda.current_stream(dev) if stream is None else stream
    check(lib().ultima_hsamp_lm_head(ctypes.byref(h), ctypes.c_void_p(s.cuda_stream)), "lm_head")
    return logits, normed


class Sampler:
    """A handle on one device (create/destroy of the C ABI)."""

    def __init__(self, device: int = 0, max_rows: int = 1024, max_vocab: int = 1 << 18):
        self.device = device
        h = ctypes.c_void_p()
        check(lib().ultima_hsamp_create(device, max_rows, max_vocab, ctypes.byref(h)), "create")
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib().ultima_hsamp_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def run(self, logits, params, u, hist=None, hist_len=None, mask=None, bias=None,
            writeback=False, want_sets=False, set_cap=None, stream=None, outputs=None, stream_only=False,
            hist_len_dev=None):
        """Sample every row. logits: cuda tensor [B, >=V] float32 or bfloat16
        (row stride = logits.stride(0)); u: cuda float64 [B]; hist: cuda int32
        [B, H]; mask: cuda int32/uint32 [B, W]. Returns a dict of cuda tensors.
        `outputs` may carry preallocated tensors (token, row_flags, ...).
        stream_only (diagnostics): run only the pass over the logits.
        hist_len_dev: cuda int32 [B], the rows' history lengths read on the
        device (a history kept by history_push)."""
        b, out, keep, s = _batch(logits, params, u, hist, hist_len, mask, bias, writeback, want_sets, set_cap,
                                 stream, outputs, stream_only, hist_len_dev)
        check(lib().ultima_hsamp_run(self.h, ctypes.byref(b), ctypes.c_void_p(s.cuda_stream)), "run")
        del keep
        return out

    def batch(self, logits, params, u, hist=None, hist_len=None, mask=None, bias=None, outputs=None):
        """The ultima_hsamp_batch run() would pass for these tensors: (batch,
        host arrays it points into, which the caller keeps alive). For callers
        that time the C ABI itself (bench.py's uncaptured figure)."""
        b, out, keep, s = _batch(logits, params, u, hist, hist_len, mask, bias, False, False, None, None,
                                 outputs, False)
        return b, (out, keep)

    def read_probe(self, logits, params, u, out, hist=None, hist_len=None, mask=None, stream=None):
        """Diagnostics: a plain read of `logits` with the launch shape run()
        would use (ultima_hsamp_read_probe); out: cuda float32, rows * 256."""
        import torch
        b, _, keep, s = _batch(logits, params, u, hist, hist_len, mask, None, False, False, None, stream,
                               {"token": out, "row_flags": out}, False)
        check(lib().ultima_hsamp_read_probe(self.h, ctypes.byref(b), ctypes.c_void_p(out.data_ptr()),
                                            ctypes.c_void_p(s.cuda_stream)), "read_probe")
        del keep, torch

    def query_kernels(self, logits, params, u, hist=None, hist_len=None, mask=None, bias=None,
                      writeback=False) -> int:
        """ultima_hsamp_query_kernels: the KERNELS_* bits of the kernels run()
        would launch for this batch (nothing is launched)."""
        b, _, keep, _s = _batch(logits, params, u, hist, hist_len, mask, bias, writeback, False, None, None,
                                None, False)
        k = ctypes.c_uint32(0)
        check(lib().ultima_hsamp_query_kernels(self.h, ctypes.byref(b), ctypes.byref(k)), "query_kernels")
        del keep
        return int(k.value)

    def set_phase_event(self, event):
        """Record `event` (a torch.cuda.Event already recorded once, or None)
        between the stream and merge kernels of every later run()."""
        ptr = None if event is None else ctypes.c_void_p(event.cuda_event)
        check(lib().ultima_hsamp_set_phase_event(self.h, ptr), "set_phase_event")

    def run_commit(self, logits, params, u, hist, hist_len, hist_len_dev, active, keep: int, stop_ids=(),
                   budget=None, mask=None, bias=None, outputs=None, stream=None):
        """ultima_hsamp_run_commit: run() over the rows' device histories
        (hist int32 [rows, stride], hist_len_dev int32 [rows]) with
        decode_commit's rules applied where each token is decided."""
        import torch
        b, out, keep_alive, s = _batch(logits, params, u, hist, hist_len, mask, bias, False, False, None, stream,
                                       outputs, False, hist_len_dev=hist_len_dev)
        stop = np.asarray(list(stop_ids), np.int32)
        c = Commit()
        c.hist, c.hist_stride, c.hist_len_dev = hist.data_ptr(), hist.stride(0), hist_len_dev.data_ptr()
        c.active = active.data_ptr()
        c.budget = budget.data_ptr() if budget is not None else None
        c.keep, c.n_stop = int(keep), int(stop.size)
        c.stop_ids = stop.ctypes.data if stop.size else None
        check(lib().ultima_hsamp_run_commit(self.h, ctypes.byref(b), ctypes.byref(c), ctypes.c_void_p(s.cuda_stream)),
              "run_commit")
        self._keep = (keep_alive, stop)
        return out

    def verify_block(self, logits, params: dict, u, draft=None, hist=None, mask=None, bias=None, stream=None):
        """ultima_hsamp_verify_block on torch tensors of one device: logits
        [n_pos, V] (each position's target logits), u f64 [n_pos], draft int32
        [n_pos - 1], hist int32 [hist_len] (the sequence's ids before the
        block), one knob dict. Returns (tokens int32 [n_pos], count int32 [1],
        row_flags int32 [n_pos]): the loop's emitted tokens are tokens[:count]."""
        import torch
        n, V = logits.shape[0], logits.shape[1]
        dev = logits.device
        dt = {torch.float32: F32, torch.bfloat16: BF16}[logits.dtype]
        assert logits.stride(1) == 1 and u.dtype == torch.float64 and u.shape[0] >= n
        assert draft is None or (draft.dtype == torch.int32 and draft.shape[0] >= n - 1)
        assert hist is None or hist.dtype == torch.int32
        L = 0 if hist is None else int(hist.shape[0])
        arr, bids, bvals = make_params([params], None, None if bias is None else [bias])
        work = torch.empty(int(lib().ultima_hsamp_verify_work_ints(n, L)), dtype=torch.int32, device=dev)
        toks = torch.empty(n, dtype=torch.int32, device=dev)
        count = torch.empty(1, dtype=torch.int32, device=dev)
        flags = torch.empty(n, dtype=torch.int32, device=dev)
        v = Verify()
        v.n_pos, v.vocab, v.dtype = n, V, dt
        v.logits, v.logits_stride = logits.data_ptr(), logits.stride(0)
        v.draft = draft.data_ptr() if draft is not None and n > 1 else None
        v.hist = hist.data_ptr() if L > 0 else None
        v.hist_len = L
        if mask is not None:
            v.mask, v.mask_stride = mask.data_ptr(), mask.stride(0)
        v.u = u.data_ptr()
        v.params = arr
        v.bias_ids = bids.ctypes.data if bids is not None else None
        v.bias_vals = bvals.ctypes.data if bvals is not None else None
        v.work, v.out_tokens, v.out_count, v.row_flags = work.data_ptr(), toks.data_ptr(), count.data_ptr(), flags.data_ptr()
        s = torch.cuda.current_stream(dev) if stream is None else stream
        check(lib().ultima_hsamp_verify_block(self.h, ctypes.byref(v), ctypes.c_void_p(s.cuda_stream)), "verify_block")
        self._keep = (arr, bids, bvals, work)   # read on the host during the call only; work until it completes
        return toks, count, flags

    def sample_host(self, logits: np.ndarray, params: dict, hist=None, bias=None, u: float = 0.5,
                    writeback: bool = False):
        """One host row (sample() with an explicit uniform). Returns (token, logits)."""
        x = np.array(logits, dtype=np.float32, copy=True)
        h = None if hist is None else np.ascontiguousarray(hist, dtype=np.int32)
        parr, bids, bvals = make_params([params], [0 if h is None else h.size], [bias] if bias else None)
        tok = ctypes.c_int32(-1)
        check(lib().ultima_hsamp_sample_host(
            self.h, x.ctypes.data, x.size, parr, None if h is None else h.ctypes.data,
            None if bids is None else bids.ctypes.data, None if bvals is None else bvals.ctypes.data,
            float(u), 1 if writeback else 0, ctypes.byref(tok)), "sample_host")
        return int(tok.value), x
