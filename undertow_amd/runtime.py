"""ctypes binding of libundertow_hip.so (the C ABI in include/undertow_hip.h).

Host-side mirror of the reference's interfaces for the decode hot path:
``QTensor`` (undertow-quant/src/qtensor.rs), the DeepSeek router
(adapters/undertow-deepseek-moe/src/router.rs), the expert store
(undertow-core/src/store.rs), ``argmax`` (undertow-core/src/sample.rs) and
the model / session / MTP loop (adapters/undertow-deepseek-moe/src/
{model,mtp}.rs).  Device buffers are torch tensors on the HIP device; the
library runs on torch's current stream so ordering with torch work is
automatic.

There is no CPU fallback: every call goes through the HIP library, and a
missing library raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
# Always the in-tree build (undertow_amd/_build.py writes it).
LIB_PATH = HERE / "lib" / "libundertow_hip.so"

F32, INT8, INT4, INFER = 0, 1, 2, -1

UT_OK = 0
UT_ERR_ARG = -1
UT_ERR_SHAPE = -2
UT_ERR_FORMAT = -3
UT_ERR_OOM = -4
UT_ERR_HIP = -5
UT_ERR_BAD_EXPERT = -6
UT_ERR_CONTEXT_OVERFLOW = -7
UT_ERR_BAD_TOKEN = -8
UT_ERR_NOT_FOUND = -9
UT_ERR_STATE = -10
UT_ERR_IO = -11


class UtError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class ShapeError(UtError, AssertionError):
    """The reference panics (assert_eq!) on a shape mismatch."""


class ContextOverflow(UtError):
    """EngineError::ContextOverflow (undertow-core/src/error.rs)."""


_vp = C.c_void_p
_i32 = C.c_int32
_i64 = C.c_int64
_f32 = C.c_float

# (name, restype, argtypes) for every symbol the header declares.
_SIGS = [
    ("ut_ctx_create", _i32, [_i32, C.POINTER(_vp)]),
    ("ut_ctx_destroy", None, [_vp]),
    ("ut_last_error", C.c_char_p, [_vp]),
    ("ut_ctx_set_stream", _i32, [_vp, _vp]),
    ("ut_ctx_stream", _vp, [_vp]),
    ("ut_ctx_synchronize", _i32, [_vp]),
    ("ut_ctx_enable_timing", _i32, [_vp, _i32]),
    ("ut_ctx_kernel_time", _i32, [_vp, C.c_char_p, C.POINTER(_i64), C.POINTER(C.c_double)]),
    ("ut_probe_read_bandwidth", _i32, [_vp, _vp, _i64, _i32, C.POINTER(C.c_double)]),
    ("ut_probe_read_windows", _i32, [_vp, _vp, _i64, _i64, _i32, C.POINTER(C.c_double)]),
    ("ut_qtensor_upload", _i32, [_vp, _i32, _vp, _i64, _vp, _i64, _i64, _i64, C.POINTER(_vp)]),
    ("ut_qtensor_free", None, [_vp]),
    ("ut_qtensor_format", _i32, [_vp]),
    ("ut_qtensor_out_dim", _i64, [_vp]),
    ("ut_qtensor_in_dim", _i64, [_vp]),
    ("ut_qtensor_nbytes", _i64, [_vp]),
    ("ut_qtensor_dequantize", _i32, [_vp, _vp, _vp]),
    ("ut_qtensor_quantize", _i32, [_vp, _i32, _vp, _i64, _i64, C.POINTER(_vp)]),
    ("ut_qtensor_download", _i32, [_vp, _vp, _vp, _i64, _vp]),
    ("ut_qtensor_matmul", _i32, [_vp, _vp, _vp, _i64, _vp, _i64, _i64]),
    ("ut_qtensor_add_scaled_row", _i32, [_vp, _vp, _i64, _f32, _vp]),
    ("ut_set_fast_int8", _i32, [_vp, _i32]),
    ("ut_fast_int8_enabled", _i32, [_vp]),
    ("ut_qtensor_matvec_rows", _i32, [_vp, _vp, _i64, _i64, _vp, _i64, _vp, _i64]),
    ("ut_route", _i32, [_vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _i32, _f32, _vp, _vp]),
    ("ut_expert_table_create", _i32, [_vp, _i64, _i64, _i64, C.POINTER(_vp)]),
    ("ut_expert_table_set", _i32, [_vp, _i64, _vp, _vp, _vp]),
    ("ut_expert_table_free", None, [_vp]),
    ("ut_moe_experts", _i32, [_vp, _vp, _vp, _vp, _i64, _i32, _vp, _vp]),
    ("ut_moe_experts_noalloc", _i32, [_vp, _vp, _vp, _vp, _i64, _i32, _vp, _vp]),
    ("ut_moe_route_experts", _i32, [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _f32, _vp,
                                    _vp, _vp, _vp]),
    ("ut_moe_experts_bf16", _i32, [_vp, _vp, _vp, _vp, _i64, _i32, _vp, _vp]),
    ("ut_moe_route_experts_bf16", _i32, [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _f32,
                                         _vp, _vp, _vp, _vp]),
    ("ut_argmax_rows", _i32, [_vp, _vp, _i64, _i64, _vp]),
    ("ut_mla_attend", _i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _f32, _vp]),
    ("ut_mla_cache_split", _i32, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    ("ut_mla_attend_split", _i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _f32, _vp]),
    ("ut_model_create", _i32, [_vp, _vp, C.POINTER(_vp)]),
    ("ut_model_set_tensor", _i32, [_vp, C.c_char_p, _i32, _vp, _i64, _vp, _i64, _i64]),
    ("ut_model_finalize", _i32, [_vp]),
    ("ut_model_load_dir", _i32, [_vp, C.c_char_p, C.POINTER(_i64)]),
    ("ut_model_load_dir_tiered", _i32, [_vp, C.c_char_p, _vp, C.POINTER(_i64)]),
    ("ut_model_synthesize_tiered", _i32, [_vp, C.c_uint64, _f32, _i32, _i32, _vp, _i64]),
    ("ut_model_pin_experts", _i32, [_vp, _vp, _i64, _i64, C.POINTER(_i64)]),
    ("ut_model_store_stats", _i32, [_vp, _vp]),
    ("ut_model_expert_usage", _i32, [_vp, _vp, _i64]),
    ("ut_model_synthesize", _i32, [_vp, C.c_uint64, _f32, _i32, _i32]),
    ("ut_model_device_bytes", _i64, [_vp]),
    ("ut_model_free", None, [_vp]),
    ("ut_session_create", _i32, [_vp, _i32, C.POINTER(_vp)]),
    ("ut_session_create_on", _i32, [_vp, _vp, _i32, C.POINTER(_vp)]),
    ("ut_model_synthesize_ex", _i32, [_vp, C.c_uint64, _f32, _i32, _i32, _i32]),
    ("ut_model_set_kv_budget", _i32, [_vp, _i64]),
    ("ut_model_max_context", _i64, [_vp]),
    ("ut_session_free", None, [_vp]),
    ("ut_session_prefill", _i32, [_vp, _vp, _i64, _vp, _vp]),
    ("ut_session_truncate", _i32, [_vp, _i64]),
    ("ut_session_position", _i64, [_vp]),
    ("ut_model_set_stop_ids", _i32, [_vp, _vp, _i64]),
    ("ut_model_enable_graphs", _i32, [_vp, _i32]),
    ("ut_model_graph_stats", _i32, [_vp, _vp, _vp, _vp]),
    ("ut_generate", _i64, [_vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp]),
    ("ut_generate_greedy", _i64, [_vp, _vp, _i64, _i64, _vp]),
    ("ut_speculative_loop", _i64, [_vp, _vp, _i64, _i64, _i32, _vp, _i64, _vp, _vp, _vp, _vp, _vp,
                                   C.POINTER(_i64), C.POINTER(_i64)]),
    ("ut_generate_mtp", _i64, [_vp, _vp, _i64, _i64, _i32, _vp, C.POINTER(_i64), C.POINTER(_i64)]),
    ("ut_session_draft_logits", _i32, [_vp, _i32, _vp, _vp]),
]

# on_token / draft_fn callbacks of the generation loops (ut_token_fn, ut_draft_fn)
TOKEN_FN = C.CFUNCTYPE(_i32, _vp, _i32)
DRAFT_FN = C.CFUNCTYPE(_i32, _vp, C.POINTER(_i32), _i64, _i32, _i32, C.POINTER(_i32))

EXPORTED = [s[0] for s in _SIGS]

_lib = None


def lib():
    """Load the built library (raises when it was never built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP backend first "
                "(python -c 'import __graft_entry__ as g; g.build()')")
        L = C.CDLL(str(LIB_PATH))
        for name, res, args in _SIGS:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


class ModelConfig(C.Structure):
    """ut_model_config: the DeepseekConfig fields the forward pass reads."""

    _fields_ = [
        ("vocab_size", _i64), ("hidden_size", _i64), ("intermediate_size", _i64),
        ("moe_intermediate_size", _i64), ("num_hidden_layers", _i64),
        ("first_k_dense_replace", _i64), ("num_attention_heads", _i64),
        ("n_routed_experts", _i64), ("num_experts_per_tok", _i64), ("n_shared_experts", _i64),
        ("n_group", _i64), ("topk_group", _i64),
        ("norm_topk_prob", _i32), ("routed_scaling_factor", _f32),
        ("q_lora_rank", _i64), ("kv_lora_rank", _i64), ("qk_nope_head_dim", _i64),
        ("qk_rope_head_dim", _i64), ("v_head_dim", _i64),
        ("rms_norm_eps", _f32), ("rope_theta", _f32),
        ("mtp", _i32), ("max_position_embeddings", _i64),
    ]

    @classmethod
    def from_dict(cls, d: dict) -> "ModelConfig":
        c = cls()
        for k, _ in cls._fields_:
            if k in d:
                setattr(c, k, d[k])
        return c


class StoreConfig(C.Structure):
    """ut_expert_store_config: cache budget, CachePolicy, pilot prefetch."""
    _fields_ = [("hbm_budget_bytes", _i64), ("policy", _i32), ("prefetch", _i32)]


class StoreStats(C.Structure):
    """ut_store_stats (StoreStatsSnapshot)."""
    _fields_ = [("hits", _i64), ("misses", _i64), ("bytes_read", _i64), ("evictions", _i64),
                ("prefetch_issued", _i64), ("prefetch_dropped", _i64), ("bytes_used", _i64),
                ("budget_bytes", _i64), ("pinned_experts", _i64), ("read_seconds", C.c_double)]

    def as_dict(self) -> dict:
        return {k: getattr(self, k) for k, _ in self._fields_}


LRU, WEIGHTED = 0, 1
SYNTH_MTP_RESTATES = 1  # ut_model_synthesize_ex: the MTP module restates a layer


class ExpertProfile:
    """ExpertProfile (undertow-core/src/profile.rs:18-100): a hot-expert
    histogram as JSON {version, architecture, counts: [[layer, expert, count]]},
    counts sorted by count descending, then layer, then expert."""

    VERSION = 1

    def __init__(self, architecture: str, counts):
        self.version = self.VERSION
        self.architecture = architecture
        self.counts = sorted(((int(l), int(e), int(c)) for l, e, c in counts),
                             key=lambda t: (-t[2], t[0], t[1]))

    @classmethod
    def from_usage(cls, architecture: str, usage) -> "ExpertProfile":
        u = np.asarray(usage)
        return cls(architecture, [(l, e, u[l, e]) for l in range(u.shape[0])
                                  for e in range(u.shape[1]) if u[l, e] > 0])

    def save(self, path) -> None:
        import json
        Path(path).write_text(json.dumps({"version": self.version, "architecture": self.architecture,
                                          "counts": [list(t) for t in self.counts]}, indent=2))

    @classmethod
    def load(cls, path) -> "ExpertProfile":
        import json
        d = json.loads(Path(path).read_text())
        if d.get("version") != cls.VERSION:
            raise ValueError(f"{path}: profile version {d.get('version')} unsupported "
                             f"(expected {cls.VERSION})")
        return cls(d["architecture"], d["counts"])

    def merge(self, other: "ExpertProfile") -> None:
        if other.architecture != self.architecture:
            raise ValueError(f"cannot merge profile for architecture '{other.architecture}' "
                             f"into '{self.architecture}'")
        acc = {}
        for l, e, c in self.counts + other.counts:
            acc[(l, e)] = acc.get((l, e), 0) + c
        self.counts = ExpertProfile(self.architecture, [(l, e, c) for (l, e), c in acc.items()]).counts

    def hottest(self):
        return [(l, e) for l, e, _ in self.counts]


def _ptr(t) -> Optional[int]:
    """Device address of a torch tensor (or None)."""
    if t is None:
        return None
    return t.data_ptr()


def _torch():
    import torch
    return torch


class Context:
    """A ut_ctx bound to torch's current stream on `device`."""

    def __init__(self, device: int = 0, bind_torch_stream: bool = True):
        s = None
        if bind_torch_stream:
            # torch's HIP runtime first: it does not come up in a process
            # where another runtime initialised the device before it
            torch = _torch()
            s = torch.cuda.current_stream(device).cuda_stream  # 0: the null stream
        h = _vp()
        rc = lib().ut_ctx_create(device, C.byref(h))
        if rc != UT_OK:
            raise UtError(rc, f"ut_ctx_create({device}) failed")
        self._h = h
        self.device = device
        self.own_stream = lib().ut_ctx_stream(self._h)
        if bind_torch_stream:
            self.check(lib().ut_ctx_set_stream(self._h, s))

    def __del__(self):
        # the library reference-counts contexts, models and sessions, so
        # finalizers may run in any order (objects in a reference cycle)
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.ut_ctx_destroy(h)
            self._h = None

    @property
    def handle(self):
        return self._h

    def last_error(self) -> str:
        return lib().ut_last_error(self._h).decode()

    def check(self, rc: int) -> int:
        if rc < 0:
            msg = self.last_error()
            if rc == UT_ERR_SHAPE:
                raise ShapeError(rc, msg)
            if rc == UT_ERR_CONTEXT_OVERFLOW:
                raise ContextOverflow(rc, msg)
            raise UtError(rc, msg)
        return rc

    def synchronize(self) -> None:
        self.check(lib().ut_ctx_synchronize(self._h))

    def enable_timing(self, on: bool) -> None:
        self.check(lib().ut_ctx_enable_timing(self._h, int(on)))

    def set_fast_int8(self, enabled: bool) -> None:
        """set_fast_int8 (undertow-quant/src/lib.rs:37-39), for this context:
        int8 QTensor matmuls quantise their activations to i8."""
        self.check(lib().ut_set_fast_int8(self._h, int(enabled)))

    def fast_int8_enabled(self) -> bool:
        return bool(lib().ut_fast_int8_enabled(self._h))

    def probe_read_bandwidth(self, buf, reps: int = 10) -> float:
        """GB/s of a plain non-temporal read of the device tensor `buf`."""
        g = C.c_double()
        self.check(lib().ut_probe_read_bandwidth(self._h, _ptr(buf), buf.numel() * buf.element_size(),
                                                 reps, C.byref(g)))
        return g.value

    def probe_read_windows(self, buf, window_bytes: int, reps: int = 16) -> float:
        """GB/s of one read launch per fresh window_bytes window of `buf`."""
        g = C.c_double()
        self.check(lib().ut_probe_read_windows(self._h, _ptr(buf), buf.numel() * buf.element_size(),
                                               window_bytes, reps, C.byref(g)))
        return g.value

    def kernel_time(self, prefix: str):
        n = _i64()
        ms = C.c_double()
        self.check(lib().ut_ctx_kernel_time(self._h, prefix.encode(), C.byref(n), C.byref(ms)))
        return n.value, ms.value


class QTensor:
    """Device QTensor (undertow-quant/src/qtensor.rs:53-71)."""

    def __init__(self, ctx: Context, fmt: int, payload, scales, out_dim: int, in_dim: int):
        """payload / scales: numpy arrays (host) or contiguous torch tensors (device)."""
        h = _vp()
        if hasattr(payload, "data_ptr"):
            p_ptr, p_len = payload.data_ptr(), payload.numel() * payload.element_size()
            s_ptr = None if scales is None else scales.data_ptr()
            s_len = 0 if scales is None else scales.numel()
            keep = (payload, scales)
        else:
            payload = np.ascontiguousarray(payload)
            sc = None if scales is None else np.ascontiguousarray(scales, np.float32)
            p_ptr, p_len = payload.ctypes.data, payload.nbytes
            s_ptr = None if sc is None else sc.ctypes.data
            s_len = 0 if sc is None else sc.size
            keep = (payload, sc)
        rc = lib().ut_qtensor_upload(ctx.handle, fmt, p_ptr, p_len, s_ptr, s_len, out_dim, in_dim,
                                     C.byref(h))
        del keep
        ctx.check(rc)
        self._h = h
        self.ctx = ctx

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.ut_qtensor_free(h)
            self._h = None

    @classmethod
    def quantize(cls, ctx: Context, w, fmt: int) -> "QTensor":
        """QTensor::quantize (qtensor.rs:142-213) of a device f32 matrix [out, in]."""
        out_dim, in_dim = w.shape
        h = _vp()
        ctx.check(lib().ut_qtensor_quantize(ctx.handle, fmt, _ptr(w), out_dim, in_dim, C.byref(h)))
        q = cls.__new__(cls)
        q._h = h
        q.ctx = ctx
        return q

    def download(self):
        """(payload uint8 array, scales float32 array | None) copied to the host."""
        fmt, o, i = self.format, self.out_dim, self.in_dim
        nb = self.nbytes - (0 if fmt == F32 else o * 4)
        payload = np.zeros(nb, np.uint8)
        scales = None if fmt == F32 else np.zeros(o, np.float32)
        self.ctx.check(lib().ut_qtensor_download(self.ctx.handle, self._h, payload.ctypes.data, nb,
                                                 None if scales is None else scales.ctypes.data))
        return payload, scales

    @property
    def handle(self):
        return self._h

    @property
    def format(self) -> int:
        return lib().ut_qtensor_format(self._h)

    @property
    def out_dim(self) -> int:
        return lib().ut_qtensor_out_dim(self._h)

    @property
    def in_dim(self) -> int:
        return lib().ut_qtensor_in_dim(self._h)

    @property
    def nbytes(self) -> int:
        return lib().ut_qtensor_nbytes(self._h)

    def dequantize(self):
        torch = _torch()
        out = torch.empty((self.out_dim, self.in_dim), dtype=torch.float32,
                          device=f"cuda:{self.ctx.device}")
        self.ctx.check(lib().ut_qtensor_dequantize(self.ctx.handle, self._h, _ptr(out)))
        return out

    def matmul(self, out, x, seq: int) -> None:
        """QTensor::matmul(&self, out, x, seq): out [seq,out_dim] <- x [seq,in_dim]."""
        self.ctx.check(lib().ut_qtensor_matmul(self.ctx.handle, self._h, _ptr(out), out.numel(),
                                               _ptr(x), x.numel(), seq))

    def matvec(self, out, x) -> None:
        self.matmul(out, x, 1)

    def add_scaled_row(self, row: int, factor: float, acc) -> None:
        self.ctx.check(lib().ut_qtensor_add_scaled_row(self.ctx.handle, self._h, row, factor,
                                                       _ptr(acc)))

    def matvec_rows(self, row0: int, nrows: int, x, out) -> None:
        """QTensor::matvec_rows: out [nrows] <- rows [row0, row0+nrows) . x [in_dim]."""
        self.ctx.check(lib().ut_qtensor_matvec_rows(self.ctx.handle, self._h, row0, nrows,
                                                    _ptr(x), x.numel(), _ptr(out), out.numel()))


def route(ctx: Context, logits, bias, top_k: int, n_group: int, topk_group: int,
          norm_topk_prob: bool, routed_scaling_factor: float):
    """DeepseekSigmoidRouter::route per row of logits [rows, E] -> (ids, weights)."""
    torch = _torch()
    rows, E = logits.shape
    ids = torch.empty((rows, top_k), dtype=torch.int32, device=logits.device)
    w = torch.empty((rows, top_k), dtype=torch.float32, device=logits.device)
    ctx.check(lib().ut_route(ctx.handle, _ptr(logits), _ptr(bias), rows, E, top_k, n_group,
                             topk_group, int(norm_topk_prob), routed_scaling_factor, _ptr(ids),
                             _ptr(w)))
    return ids, w


def argmax_rows(ctx: Context, logits):
    torch = _torch()
    rows, V = logits.shape
    idx = torch.empty(rows, dtype=torch.int32, device=logits.device)
    ctx.check(lib().ut_argmax_rows(ctx.handle, _ptr(logits), rows, V, _ptr(idx)))
    return idx


def mla_attend(ctx: Context, qabs, q_rope, latent, krot, pos_base: int, scale: float, out=None):
    torch = _torch()
    R, H, L = qabs.shape
    P = q_rope.shape[2]
    if out is None:
        out = torch.empty((R, H, L), dtype=torch.float32, device=qabs.device)
    elif tuple(out.shape) != (R, H, L) or out.dtype != torch.float32 or not out.is_contiguous():
        raise ShapeError(f"mla_attend: out must be a contiguous float32 [{R}, {H}, {L}] tensor")
    ctx.check(lib().ut_mla_attend(ctx.handle, _ptr(qabs), _ptr(q_rope), _ptr(latent), _ptr(krot),
                                  R, H, L, P, pos_base, scale, _ptr(out)))
    return out


def mla_cache_split(ctx: Context, latent, krot):
    """The cache [T, L] + [T, P] (f32) in the split bf16 form of the MFMA
    attention kernel: an int16 tensor [T, 2, L + P] (hi parts, then lo)."""
    torch = _torch()
    T, L = latent.shape
    P = krot.shape[1]
    kc = torch.empty((T, 2, L + P), dtype=torch.int16, device=latent.device)
    ctx.check(lib().ut_mla_cache_split(ctx.handle, _ptr(latent), _ptr(krot), T, L, P, _ptr(kc)))
    return kc


def mla_attend_split(ctx: Context, qabs, q_rope, kc, pos_base: int, scale: float, out=None):
    torch = _torch()
    R, H, L = qabs.shape
    P = q_rope.shape[2]
    if kc.shape[-1] != L + P:
        raise ShapeError(f"mla_attend_split: cache width {kc.shape[-1]} != {L} + {P}")
    if out is None:
        out = torch.empty((R, H, L), dtype=torch.float32, device=qabs.device)
    ctx.check(lib().ut_mla_attend_split(ctx.handle, _ptr(qabs), _ptr(q_rope), _ptr(kc), R, H, L, P,
                                        pos_base, scale, _ptr(out)))
    return out


class ExpertTable:
    """Device expert store for one MoE layer (keeps its QTensors alive)."""

    def __init__(self, ctx: Context, n_experts: int, hidden: int, inter: int):
        h = _vp()
        ctx.check(lib().ut_expert_table_create(ctx.handle, n_experts, hidden, inter, C.byref(h)))
        self._h = h
        self.ctx = ctx
        self._keep = {}

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.ut_expert_table_free(h)
            self._h = None

    def set(self, e: int, gate: QTensor, up: QTensor, down: QTensor) -> None:
        self.ctx.check(lib().ut_expert_table_set(self._h, e, gate.handle, up.handle, down.handle))
        self._keep[e] = (gate, up, down)

    def moe_experts(self, ids, weights, x):
        """The routed experts over f32 or bf16 activations x [rows, hidden];
        the result is f32 either way."""
        torch = _torch()
        rows, k = ids.shape
        out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
        fn = lib().ut_moe_experts_bf16 if x.dtype == torch.bfloat16 else lib().ut_moe_experts
        self.ctx.check(fn(self.ctx.handle, self._h, _ptr(ids), _ptr(weights), rows, k, _ptr(x),
                          _ptr(out)))
        return out

    def moe_experts_noalloc(self, ids, weights, x, out) -> None:
        """ut_moe_experts into a caller's `out`, allocating nothing."""
        rows, k = ids.shape
        self.ctx.check(lib().ut_moe_experts_noalloc(self.ctx.handle, self._h, _ptr(ids),
                                                    _ptr(weights), rows, k, _ptr(x), _ptr(out)))

    def moe_route_experts(self, logits, bias, x, k, n_group, topk_group, norm_topk_prob,
                          routed_scaling_factor):
        """Route (ut_route's semantics) and run the experts in one call;
        returns (out, ids, weights).  x may be f32 or bf16; out is f32."""
        torch = _torch()
        rows = x.shape[0]
        out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
        ids = torch.empty((rows, k), dtype=torch.int32, device=x.device)
        w = torch.empty((rows, k), dtype=torch.float32, device=x.device)
        fn = (lib().ut_moe_route_experts_bf16 if x.dtype == torch.bfloat16
              else lib().ut_moe_route_experts)
        self.ctx.check(fn(
            self.ctx.handle, self._h, _ptr(logits), _ptr(bias) if bias is not None else None, rows,
            k, n_group, topk_group, int(norm_topk_prob), routed_scaling_factor, _ptr(x), _ptr(out),
            _ptr(ids), _ptr(w)))
        return out, ids, w


class Model:
    """DeepseekMoeModel on device (adapters/undertow-deepseek-moe/src/model.rs)."""

    def __init__(self, ctx: Context, cfg: dict):
        self.ctx = ctx
        self.cfg = dict(cfg)
        self._cfg = ModelConfig.from_dict(cfg)
        h = _vp()
        ctx.check(lib().ut_model_create(ctx.handle, C.byref(self._cfg), C.byref(h)))
        self._h = h

    def _release(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.ut_model_free(h)
        self._h = None

    def __del__(self):
        self._release()

    def set_tensor(self, name: str, fmt: int, payload: np.ndarray, scales, shape) -> None:
        payload = np.ascontiguousarray(payload)
        sc = None if scales is None else np.ascontiguousarray(scales, np.float32)
        d0 = shape[0]
        d1 = shape[1] if len(shape) == 2 else 1
        self.ctx.check(lib().ut_model_set_tensor(self._h, name.encode(), fmt, payload.ctypes.data,
                                                 payload.nbytes,
                                                 None if sc is None else sc.ctypes.data, d0, d1))

    def finalize(self) -> None:
        self.ctx.check(lib().ut_model_finalize(self._h))

    def load_dir_tiered(self, path, hbm_budget_bytes: int, policy: int = LRU,
                        prefetch: bool = False) -> int:
        """Dense tensors into HBM, routed experts behind the HBM tier of the
        expert store; returns the bytes read at load."""
        cfg = StoreConfig(hbm_budget_bytes, policy, int(prefetch))
        n = _i64()
        self.ctx.check(lib().ut_model_load_dir_tiered(self._h, str(path).encode(), C.byref(cfg),
                                                      C.byref(n)))
        return n.value

    def synthesize_tiered(self, seed: int, hbm_budget_bytes: int, host_pool_experts: int,
                          init_std: float = 0.02, expert_fmt: int = INT4, dense_fmt: int = INT8,
                          policy: int = LRU, prefetch: bool = False) -> None:
        cfg = StoreConfig(hbm_budget_bytes, policy, int(prefetch))
        self.ctx.check(lib().ut_model_synthesize_tiered(self._h, seed, init_std, expert_fmt,
                                                        dense_fmt, C.byref(cfg), host_pool_experts))

    def pin_experts(self, keys, budget_bytes: int) -> int:
        """pin_hottest over (layer, expert) keys; returns the pinned bytes."""
        a = np.ascontiguousarray(np.asarray(keys, np.int32).reshape(-1, 2))
        n = _i64()
        self.ctx.check(lib().ut_model_pin_experts(self._h, a.ctypes.data if a.size else None,
                                                  a.shape[0], budget_bytes, C.byref(n)))
        return n.value

    def store_stats(self) -> dict:
        st = StoreStats()
        self.ctx.check(lib().ut_model_store_stats(self._h, C.byref(st)))
        return st.as_dict()

    def expert_usage(self) -> np.ndarray:
        L = self.cfg["num_hidden_layers"] + (1 if self.cfg.get("mtp") else 0)
        E = self.cfg["n_routed_experts"]
        u = np.zeros((L, E), np.int64)
        self.ctx.check(lib().ut_model_expert_usage(self._h, u.ctypes.data, u.size))
        return u

    def load_dir(self, path) -> int:
        """Stream a converted checkpoint directory into HBM and finalize;
        returns the bytes read."""
        n = _i64()
        self.ctx.check(lib().ut_model_load_dir(self._h, str(path).encode(), C.byref(n)))
        return n.value

    def synthesize(self, seed: int, init_std: float = 0.02, expert_fmt: int = INT4,
                   dense_fmt: int = INT8, mtp_restates: bool = False) -> None:
        """Seeded random weights made on the device; mtp_restates: the MTP
        module restates the first MoE layer (a head that accepts drafts)."""
        self.ctx.check(lib().ut_model_synthesize_ex(self._h, seed, init_std, expert_fmt, dense_fmt,
                                                    SYNTH_MTP_RESTATES if mtp_restates else 0))

    def set_kv_budget(self, kv_budget_bytes: Optional[int]) -> None:
        """LoadOptions::kv_budget_bytes: lowers the context sessions hold
        (None removes the bound)."""
        self.ctx.check(lib().ut_model_set_kv_budget(self._h, -1 if kv_budget_bytes is None
                                                    else kv_budget_bytes))

    @property
    def max_context(self) -> int:
        return int(lib().ut_model_max_context(self._h))

    @property
    def device_bytes(self) -> int:
        return lib().ut_model_device_bytes(self._h)

    def session(self, path: int = 0, ctx: Optional[Context] = None) -> "Session":
        return Session(self, path, ctx)

    def forward(self, ids) -> np.ndarray:
        return self.session().prefill(ids)

    def set_stop_ids(self, ids) -> None:
        """DeepseekMoeModel::stop_ids (loader.rs:304-309)."""
        a = np.ascontiguousarray(ids, np.int32)
        self.ctx.check(lib().ut_model_set_stop_ids(self._h, a.ctypes.data if a.size else None,
                                                   a.size))

    def enable_graphs(self, on: bool = True) -> None:
        """Device-fed decode steps (one row) and MTP verify steps replayed
        from graphs captured per session."""
        self.ctx.check(lib().ut_model_enable_graphs(self._h, int(on)))

    def graph_stats(self) -> dict:
        c, r, f = C.c_int64(), C.c_int64(), C.c_int64()
        self.ctx.check(lib().ut_model_graph_stats(self._h, C.byref(c), C.byref(r), C.byref(f)))
        return {"captures": c.value, "replays": r.value, "failures": f.value}

    def generate_greedy(self, prompt, max_new: int) -> list:
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max(max_new, 1), np.int32)
        n = lib().ut_generate_greedy(self._h, p.ctypes.data, p.size, max_new, out.ctypes.data)
        self.ctx.check(int(n))
        return out[:n].tolist()

    def generate(self, prompt, max_new: int, extra_stop_ids=(), on_token=None) -> list:
        """undertow_core::generate, greedy: stops after a stop id (emitted),
        when on_token(id) returns False, or at max_new tokens."""
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max(max_new, 1), np.int32)
        st = np.ascontiguousarray(extra_stop_ids, np.int32)
        cb = TOKEN_FN(lambda _u, t: int(bool(on_token(t)))) if on_token else None
        n = lib().ut_generate(self._h, p.ctypes.data, p.size, max_new,
                              st.ctypes.data if st.size else None, st.size,
                              C.cast(cb, _vp) if cb else None, None, out.ctypes.data)
        self.ctx.check(int(n))
        return out[:n].tolist()

    def speculative_loop(self, prompt, max_new: int, depth: int = 1, draft_fn=None,
                         extra_stop_ids=(), on_token=None):
        """speculative_loop (mtp.rs:263-314).  draft_fn(tokens, next, depth)
        -> list of `depth` ids; None drafts with the native MTP head.
        Returns (tokens, drafted, accepted)."""
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max(max_new, 1), np.int32)
        st = np.ascontiguousarray(extra_stop_ids, np.int32)
        tcb = TOKEN_FN(lambda _u, t: int(bool(on_token(t)))) if on_token else None
        err = []

        def _draft(_u, toks, n, nxt, dep, dst):
            try:
                ids = list(draft_fn([toks[i] for i in range(n)], nxt, dep))
                for i in range(dep):
                    dst[i] = int(ids[i])
                return 0
            except Exception as e:  # surfaced after the call
                err.append(e)
                return UT_ERR_STATE

        dcb = DRAFT_FN(_draft) if draft_fn else None
        d, a = _i64(), _i64()
        n = lib().ut_speculative_loop(self._h, p.ctypes.data, p.size, max_new, depth,
                                      st.ctypes.data if st.size else None, st.size,
                                      C.cast(tcb, _vp) if tcb else None, None,
                                      C.cast(dcb, _vp) if dcb else None, None,
                                      out.ctypes.data, C.byref(d), C.byref(a))
        if err:
            raise err[0]
        self.ctx.check(int(n))
        return out[:n].tolist(), d.value, a.value

    def generate_mtp(self, prompt, max_new: int, depth: int = 1):
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max(max_new, 1), np.int32)
        d, a = _i64(), _i64()
        n = lib().ut_generate_mtp(self._h, p.ctypes.data, p.size, max_new, depth,
                                  out.ctypes.data, C.byref(d), C.byref(a))
        self.ctx.check(int(n))
        return out[:n].tolist(), d.value, a.value


class Session:
    """InferenceSession (model.rs:407-564) on device."""

    def __init__(self, model: Model, path: int = 0, ctx: Optional[Context] = None):
        """ctx: run the session's work on this context (its own stream)
        instead of the model's, so sessions on several threads can share
        one model."""
        self.model = model
        self.ctx = ctx or model.ctx
        h = _vp()
        self.ctx.check(lib().ut_session_create_on(model._h, None if ctx is None else ctx.handle,
                                                  path, C.byref(h)))
        self._h = h

    def _release(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.ut_session_free(h)
        self._h = None

    def __del__(self):
        self._release()

    def prefill(self, ids, want_logits: bool = True):
        ids = np.ascontiguousarray(ids, np.int32)
        V = self.model.cfg["vocab_size"]
        logits = np.zeros((ids.size, V), np.float32) if want_logits else None
        am = np.zeros(max(ids.size, 1), np.int32)
        rc = lib().ut_session_prefill(self._h, ids.ctypes.data, ids.size,
                                      None if logits is None else logits.ctypes.data,
                                      am.ctypes.data)
        self.ctx.check(rc)
        self.last_argmax = am[:ids.size].tolist()
        return logits

    def decode(self, tok: int):
        return self.prefill([tok])[0]

    def draft_logits(self, next_token: int):
        """draft_logits (mtp.rs:74-133) on this session's MTP state ->
        (logits [vocab], draft id)."""
        V = self.model.cfg["vocab_size"]
        logits = np.zeros(V, np.float32)
        d = _i32()
        self.ctx.check(lib().ut_session_draft_logits(self._h, next_token,
                                                     logits.ctypes.data, C.byref(d)))
        return logits, d.value

    def truncate(self, n: int) -> None:
        self.ctx.check(lib().ut_session_truncate(self._h, n))

    @property
    def position(self) -> int:
        return int(lib().ut_session_position(self._h))
