"""ctypes bindings for the CPU oracle (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module.  It is the checker, never the thing measured or shipped:
the product package ``undertow_amd`` does not import it.

The C library restates the undertow reference's scalar CPU path; see
oracle/ut_oracle.h for the function-by-function reference citations.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_DIR = HERE / "lib"

F32, INT8, INT4 = 0, 1, 2

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")


def build() -> None:
    """Compile the oracle libraries (gcc; no GPU needed)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


class Spec(C.Structure):
    """uto_spec: OracleSpec + the DeepseekConfig fields the forward reads."""

    _fields_ = [
        ("seed", C.c_uint64),
        ("vocab_size", C.c_int64), ("hidden_size", C.c_int64),
        ("intermediate_size", C.c_int64), ("moe_intermediate_size", C.c_int64),
        ("num_hidden_layers", C.c_int64), ("first_k_dense_replace", C.c_int64),
        ("num_attention_heads", C.c_int64),
        ("n_routed_experts", C.c_int64), ("num_experts_per_tok", C.c_int64),
        ("n_shared_experts", C.c_int64),
        ("n_group", C.c_int64), ("topk_group", C.c_int64),
        ("norm_topk_prob", C.c_int32),
        ("routed_scaling_factor", C.c_float),
        ("q_lora_rank", C.c_int64), ("kv_lora_rank", C.c_int64),
        ("qk_nope_head_dim", C.c_int64), ("qk_rope_head_dim", C.c_int64),
        ("v_head_dim", C.c_int64),
        ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float), ("init_std", C.c_float),
        ("mtp", C.c_int32),
        ("max_position_embeddings", C.c_int64),
    ]

    def as_dict(self) -> dict:
        return {k: getattr(self, k) for k, _ in self._fields_}


_lib = None
_cb = None
_cm = None


def lib():
    """The scalar restatement (the parity checker)."""
    global _lib
    if _lib is None:
        _lib = _load("liboracle.so")
    return _lib


def cpu_model_lib():
    """The same model code over the restated dispatched SIMD kernels
    (libcpu_model.so): the timed CPU baseline, never a parity checker."""
    global _cm
    if _cm is None:
        _cm = _load("libcpu_model.so")
    return _cm


def _load(name):
    path = LIB_DIR / name
    if not path.exists():
        build()
    L = C.CDLL(str(path))
    if True:
        L.uto_pcg32_fill.argtypes = [C.c_uint64, C.c_uint64, C.c_int, C.c_float, _f32p, C.c_int64]
        L.uto_payload_bytes.restype = C.c_int64
        L.uto_payload_bytes.argtypes = [C.c_int, C.c_int64, C.c_int64]
        L.uto_quantize.argtypes = [C.c_int, _f32p, C.c_int64, C.c_int64, C.c_void_p, _f32p]
        L.uto_dequantize.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, _f32p]
        L.uto_matmul.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, _f32p, C.c_int64, _f32p]
        L.uto_quantize_activations.argtypes = [_f32p, C.c_int64, C.c_void_p]
        L.uto_quantize_activations.restype = C.c_float
        L.uto_matmul_fast_i8.argtypes = [C.c_void_p, _f32p, C.c_int64, C.c_int64, _f32p, C.c_int64, _f32p]
        L.uto_set_fast_int8.argtypes = [C.c_int]
        L.uto_fast_int8_enabled.restype = C.c_int
        L.uto_add_scaled_row.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_float, _f32p]
        L.uto_matvec_rows.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_int64, _f32p, _f32p]
        L.uto_rmsnorm.argtypes = [_f32p, _f32p, _f32p, C.c_int64, C.c_float]
        L.uto_softmax.argtypes = [_f32p, C.c_int64]
        L.uto_sigmoid.restype = C.c_float
        L.uto_sigmoid.argtypes = [C.c_float]
        L.uto_silu.restype = C.c_float
        L.uto_silu.argtypes = [C.c_float]
        L.uto_rope_interleave.argtypes = [_f32p, C.c_int64, C.c_int64, C.c_float]
        L.uto_argmax.restype = C.c_int64
        L.uto_argmax.argtypes = [_f32p, C.c_int64]
        L.uto_topk_indices.restype = C.c_int64
        L.uto_topk_indices.argtypes = [_f32p, C.c_int64, C.c_int64, _i64p]
        L.uto_route.argtypes = [_f32p, C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_int64,
                                C.c_int, C.c_float, _i64p, _f32p]
        L.uto_moe_experts.argtypes = [C.c_int, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p,
                                      C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                      C.c_int64, C.c_int64, _i64p, _f32p, _f32p, _f32p]
        L.uto_mla_attend.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int64, C.c_int64, C.c_int64,
                                     C.c_int64, C.c_int64, C.c_float, _f32p]
        L.uto_spec_default.argtypes = [C.POINTER(Spec)]
        L.uto_generate.restype = C.c_void_p
        L.uto_generate.argtypes = [C.POINTER(Spec)]
        L.uto_ckpt_free.argtypes = [C.c_void_p]
        L.uto_ckpt_safetensors.restype = C.c_int64
        L.uto_ckpt_safetensors.argtypes = [C.c_void_p, C.c_void_p, C.c_int64]
        L.uto_ckpt_convert.argtypes = [C.c_void_p, C.c_int, C.c_int]
        L.uto_ckpt_count.restype = C.c_int64
        L.uto_ckpt_count.argtypes = [C.c_void_p]
        L.uto_ckpt_info.argtypes = [C.c_void_p, C.c_int64, C.c_char_p, C.c_int64,
                                    C.POINTER(C.c_int32), C.POINTER(C.c_int64), C.POINTER(C.c_int32)]
        L.uto_ckpt_payload.restype = C.c_void_p
        L.uto_ckpt_payload.argtypes = [C.c_void_p, C.c_int64, C.POINTER(C.c_int64)]
        L.uto_ckpt_scales.restype = C.c_void_p
        L.uto_ckpt_scales.argtypes = [C.c_void_p, C.c_int64]
        L.uto_model_new.restype = C.c_void_p
        L.uto_model_new.argtypes = [C.c_void_p, C.POINTER(Spec)]
        L.uto_model_free.argtypes = [C.c_void_p]
        L.uto_session_new.restype = C.c_void_p
        L.uto_session_new.argtypes = [C.c_void_p, C.c_int]
        L.uto_session_free.argtypes = [C.c_void_p]
        L.uto_session_prefill.argtypes = [C.c_void_p, _i32p, C.c_int64, C.c_void_p]
        L.uto_session_truncate.argtypes = [C.c_void_p, C.c_int64]
        L.uto_session_position.restype = C.c_int64
        L.uto_session_position.argtypes = [C.c_void_p]
        L.uto_greedy_decode.restype = C.c_int64
        L.uto_greedy_decode.argtypes = [C.c_void_p, _i32p, C.c_int64, C.c_int64, _i32p]
        L.uto_generate_mtp.restype = C.c_int64
        L.uto_generate_mtp.argtypes = [C.c_void_p, _i32p, C.c_int64, C.c_int64, _i32p,
                                       C.POINTER(C.c_int64), C.POINTER(C.c_int64)]
        L.uto_ckpt_new.restype = C.c_void_p
        L.uto_ckpt_new.argtypes = []
        L.uto_ckpt_add.argtypes = [C.c_void_p, C.c_char_p, C.c_int32, C.c_int32, C.c_int64,
                                   C.c_int64, C.c_void_p, C.c_int64, C.c_void_p]
        L.uto_ckpt_synthesize.restype = C.c_void_p
        L.uto_ckpt_synthesize.argtypes = [C.POINTER(Spec), C.c_uint64, C.c_float, C.c_int, C.c_int]
        L.uto_generate_greedy.restype = C.c_int64
        L.uto_generate_greedy.argtypes = [C.c_void_p, _i32p, C.c_int64, C.c_int64, C.c_void_p,
                                          C.c_int64, C.c_void_p, C.c_void_p, _i32p]
        L.uto_speculative_loop.restype = C.c_int64
        L.uto_speculative_loop.argtypes = [C.c_void_p, _i32p, C.c_int64, C.c_int64, C.c_int32,
                                           C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p,
                                           C.c_void_p, C.c_void_p, _i32p, C.POINTER(C.c_int64),
                                           C.POINTER(C.c_int64)]
        L.uto_mtp_state_new.restype = C.c_void_p
        L.uto_mtp_state_new.argtypes = []
        L.uto_mtp_state_free.argtypes = [C.c_void_p]
        L.uto_draft_logits.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, _f32p,
                                       C.c_void_p]
    return L


def cpu_baseline_lib():
    global _cb
    if _cb is None:
        path = LIB_DIR / "libcpu_baseline.so"
        if not path.exists():
            build()
        L = C.CDLL(str(path))
        L.ucb_isa.restype = C.c_int
        L.ucb_set_isa.argtypes = [C.c_int]
        L.ucb_max_threads.restype = C.c_int
        L.ucb_matmul.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, _f32p,
                                 C.c_int64, _f32p, C.c_int]
        L.ucb_moe_experts.argtypes = [C.c_int, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p,
                                      C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                      C.c_int64, C.c_int64, _i64p, _f32p, _f32p, _f32p, C.c_int]
        L.ucb_mla_attend.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int64, C.c_int64, C.c_int64,
                                     C.c_int64, C.c_int64, C.c_float, _f32p, C.c_int]
        _cb = L
    return _cb


# ----------------------------------------------------------------- helpers --

def _vp(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def payload_bytes(fmt: int, out_dim: int, in_dim: int) -> int:
    return int(lib().uto_payload_bytes(fmt, out_dim, in_dim))


def pcg32_fill(seed: int, stream: int, n: int, kind: str = "normal", std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().uto_pcg32_fill(seed, stream, 0 if kind == "uniform" else 1, std, out, n)
    return out


def quantize(w: np.ndarray, fmt: int):
    """QTensor::quantize -> (payload uint8/int8, scales).  Raises on non-finite."""
    w = np.ascontiguousarray(w, np.float32)
    o, i = w.shape
    if fmt == F32:
        return w.copy(), None
    payload = np.zeros(payload_bytes(fmt, o, i), np.uint8)
    scales = np.zeros(o, np.float32)
    if lib().uto_quantize(fmt, w, o, i, _vp(payload), scales) != 0:
        raise ValueError("non-finite weight")
    if fmt == INT8:
        payload = payload.view(np.int8).reshape(o, i)
    else:
        payload = payload.reshape(o, (i + 1) // 2)
    return payload, scales


def dequantize(fmt: int, payload: np.ndarray, scales, out_dim: int, in_dim: int) -> np.ndarray:
    out = np.zeros(out_dim * in_dim, np.float32)
    payload = np.ascontiguousarray(payload)
    sc = None if scales is None else np.ascontiguousarray(scales, np.float32)
    lib().uto_dequantize(fmt, _vp(payload), None if sc is None else _vp(sc), out_dim, in_dim, out)
    return out.reshape(out_dim, in_dim)


def matmul(fmt: int, payload: np.ndarray, scales, out_dim: int, in_dim: int, x: np.ndarray) -> np.ndarray:
    """QTensor::matmul_scalar: x [seq, in] -> [seq, out]."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, in_dim)
    seq = x.shape[0]
    out = np.zeros(seq * out_dim, np.float32)
    payload = np.ascontiguousarray(payload)
    sc = None if scales is None else np.ascontiguousarray(scales, np.float32)
    lib().uto_matmul(fmt, _vp(payload), None if sc is None else _vp(sc), out_dim, in_dim,
                     x.reshape(-1), seq, out)
    return out.reshape(seq, out_dim)


def quantize_activations(x: np.ndarray):
    """lib.rs:46-59: (i8 codes, scale) of one activation row."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    q = np.zeros(x.size, np.int8)
    s = lib().uto_quantize_activations(x, x.size, _vp(q))
    return q, np.float32(s)


def matmul_fast_i8(payload: np.ndarray, scales, out_dim: int, in_dim: int,
                   x: np.ndarray) -> np.ndarray:
    """The opt-in fast-int8 matmul (avx512.rs:221-242): x [seq, in] -> [seq, out]."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, in_dim)
    seq = x.shape[0]
    out = np.zeros(seq * out_dim, np.float32)
    q = np.ascontiguousarray(payload).view(np.int8)
    sc = np.ascontiguousarray(scales, np.float32)
    lib().uto_matmul_fast_i8(_vp(q), sc, out_dim, in_dim, x.reshape(-1), seq, out)
    return out.reshape(seq, out_dim)


def set_fast_int8(enabled: bool) -> None:
    """undertow_core::set_fast_int8 (undertow-quant/src/lib.rs:35-43): the
    oracle's int8 matmuls take the fast path while set (process-global)."""
    lib().uto_set_fast_int8(int(bool(enabled)))


def fast_int8_enabled() -> bool:
    return bool(lib().uto_fast_int8_enabled())


def add_scaled_row(fmt, payload, scales, out_dim, in_dim, row, factor, acc):
    acc = np.ascontiguousarray(acc, np.float32).copy()
    payload = np.ascontiguousarray(payload)
    sc = None if scales is None else np.ascontiguousarray(scales, np.float32)
    lib().uto_add_scaled_row(fmt, _vp(payload), None if sc is None else _vp(sc), out_dim, in_dim,
                             row, factor, acc)
    return acc


def matvec_rows(fmt, payload, scales, out_dim, in_dim, row0, nrows, x):
    out = np.zeros(nrows, np.float32)
    payload = np.ascontiguousarray(payload)
    sc = None if scales is None else np.ascontiguousarray(scales, np.float32)
    lib().uto_matvec_rows(fmt, _vp(payload), None if sc is None else _vp(sc), out_dim, in_dim,
                          row0, nrows, np.ascontiguousarray(x, np.float32), out)
    return out


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(x)
    lib().uto_rmsnorm(out, x, np.ascontiguousarray(w, np.float32), x.size, eps)
    return out


def softmax(x):
    x = np.ascontiguousarray(x, np.float32).copy()
    lib().uto_softmax(x, x.size)
    return x


def rope_interleave(v, pos, dim, theta):
    v = np.ascontiguousarray(v, np.float32).copy()
    lib().uto_rope_interleave(v, pos, dim, theta)
    return v


def argmax(v) -> int:
    v = np.ascontiguousarray(v, np.float32)
    return int(lib().uto_argmax(v, v.size))


def topk_indices(v, k):
    v = np.ascontiguousarray(v, np.float32)
    out = np.zeros(max(k, 1), np.int64)
    n = lib().uto_topk_indices(v, v.size, k, out)
    return out[:n].tolist()


def route(logits, bias, top_k, n_group, topk_group, norm_topk_prob, scale):
    logits = np.ascontiguousarray(logits, np.float32)
    ids = np.zeros(top_k, np.int64)
    w = np.zeros(top_k, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().uto_route(logits, None if b is None else _vp(b), logits.size, top_k, n_group, topk_group,
                    int(norm_topk_prob), scale, ids, w)
    return ids, w


def moe_experts(fmt, hidden, inter, gate, gate_s, up, up_s, down, down_s, ids, weights, x):
    """Routed expert block: expert e's payload at base + e*stride."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, hidden)
    M = x.shape[0]
    ids = np.ascontiguousarray(ids, np.int64).reshape(M, -1)
    k = ids.shape[1]
    out = np.zeros(M * hidden, np.float32)
    arrs = [np.ascontiguousarray(a) for a in (gate, gate_s, up, up_s, down, down_s)]
    lib().uto_moe_experts(fmt, hidden, inter, *[_vp(a) for a in arrs], M, k, ids.reshape(-1),
                          np.ascontiguousarray(weights, np.float32).reshape(-1), x.reshape(-1), out)
    return out.reshape(M, hidden)


def mla_attend(qabs, q_rope, latent, krot, pos_base, scale):
    qabs = np.ascontiguousarray(qabs, np.float32)
    q_rope = np.ascontiguousarray(q_rope, np.float32)
    R, H, L = qabs.shape
    P = q_rope.shape[2]
    out = np.zeros((R, H, L), np.float32)
    lib().uto_mla_attend(qabs.reshape(-1), q_rope.reshape(-1),
                         np.ascontiguousarray(latent, np.float32).reshape(-1),
                         np.ascontiguousarray(krot, np.float32).reshape(-1),
                         R, H, L, P, pos_base, scale, out.reshape(-1))
    return out


# ------------------------------------------------------ checkpoint / model --

def default_spec(**overrides) -> Spec:
    s = Spec()
    lib().uto_spec_default(C.byref(s))
    for k, v in overrides.items():
        setattr(s, k, v)
    return s


TOKEN_FN = C.CFUNCTYPE(C.c_int32, C.c_void_p, C.c_int32)
DRAFT_FN = C.CFUNCTYPE(C.c_int32, C.c_void_p, C.POINTER(C.c_int32), C.c_int64, C.c_int32,
                       C.c_int32, C.POINTER(C.c_int32))


class Checkpoint:
    """A generated (optionally converted) checkpoint held by the C oracle."""

    def __init__(self, spec: Spec, _handle=None, L=None):
        self.L = L or lib()
        self.spec = spec
        self._h = _handle if _handle is not None else self.L.uto_generate(C.byref(spec))

    @classmethod
    def synthesize(cls, spec: Spec, seed: int, std: float, expert_fmt: int,
                   dense_fmt: int, L=None) -> "Checkpoint":
        """Seeded weights at large widths in converted form (uto_ckpt_synthesize)."""
        L = L or lib()
        return cls(spec, L.uto_ckpt_synthesize(C.byref(spec), seed, std, expert_fmt, dense_fmt), L)

    @classmethod
    def from_tensors(cls, spec: Spec, tensors) -> "Checkpoint":
        """A checkpoint of (name, fmt, shape, payload, scales) tuples."""
        L = lib()
        h = L.uto_ckpt_new()
        ck = cls(spec, h)
        for name, fmt, shape, payload, scales in tensors:
            payload = np.ascontiguousarray(payload)
            sc = None if scales is None else np.ascontiguousarray(scales, np.float32)
            d1 = shape[1] if len(shape) == 2 else 1
            rc = L.uto_ckpt_add(h, name.encode(), fmt, len(shape), shape[0], d1,
                                payload.ctypes.data, payload.nbytes,
                                None if sc is None else sc.ctypes.data)
            if rc != 0:
                raise ValueError(f"uto_ckpt_add({name}) failed")
        return ck

    def raw_tensors(self):
        """Yield (name, fmt, shape, payload address, nbytes, scales address|None)
        without copying (valid while the checkpoint lives)."""
        L = self.L
        name = C.create_string_buffer(256)
        fmt = C.c_int32()
        shape = (C.c_int64 * 2)()
        ndim = C.c_int32()
        nb = C.c_int64()
        for i in range(L.uto_ckpt_count(self._h)):
            L.uto_ckpt_info(self._h, i, name, 256, C.byref(fmt), shape, C.byref(ndim))
            p = L.uto_ckpt_payload(self._h, i, C.byref(nb))
            shp = (shape[0], shape[1]) if ndim.value == 2 else (shape[0],)
            sp = L.uto_ckpt_scales(self._h, i) if fmt.value != F32 else None
            yield name.value.decode(), fmt.value, shp, p, nb.value, sp

    def __del__(self):
        if getattr(self, "_h", None):
            self.L.uto_ckpt_free(self._h)
            self._h = None

    def safetensors_bytes(self) -> bytes:
        n = self.L.uto_ckpt_safetensors(self._h, None, 0)
        buf = (C.c_uint8 * n)()
        self.L.uto_ckpt_safetensors(self._h, buf, n)
        return bytes(buf)

    def convert(self, expert_fmt: int, dense_fmt: int) -> None:
        if self.L.uto_ckpt_convert(self._h, expert_fmt, dense_fmt) != 0:
            raise ValueError("conversion failed (non-finite weight)")

    def tensors(self):
        """Yield (name, fmt, shape, payload ndarray, scales ndarray|None)."""
        L = self.L
        name = C.create_string_buffer(256)
        fmt = C.c_int32()
        shape = (C.c_int64 * 2)()
        ndim = C.c_int32()
        nb = C.c_int64()
        for i in range(L.uto_ckpt_count(self._h)):
            L.uto_ckpt_info(self._h, i, name, 256, C.byref(fmt), shape, C.byref(ndim))
            p = L.uto_ckpt_payload(self._h, i, C.byref(nb))
            raw = np.ctypeslib.as_array((C.c_uint8 * nb.value).from_address(p)).copy()
            shp = (shape[0], shape[1]) if ndim.value == 2 else (shape[0],)
            sc = None
            if fmt.value != F32:
                sp = L.uto_ckpt_scales(self._h, i)
                sc = np.ctypeslib.as_array((C.c_float * shape[0]).from_address(sp)).copy()
            yield name.value.decode(), fmt.value, shp, raw, sc


class Model:
    def __init__(self, ckpt: Checkpoint):
        self.ckpt = ckpt  # keeps the tensors alive
        self.spec = ckpt.spec
        self.L = ckpt.L  # the library the checkpoint was made with
        self._h = self.L.uto_model_new(ckpt._h, C.byref(ckpt.spec))
        if not self._h:
            raise ValueError("oracle model build failed")

    def __del__(self):
        if getattr(self, "_h", None):
            self.L.uto_model_free(self._h)
            self._h = None

    def session(self, path: int = 0) -> "Session":
        return Session(self, path)

    def forward(self, ids) -> np.ndarray:
        return self.session().prefill(ids)

    def greedy_decode(self, prompt, max_new: int) -> list:
        p = np.asarray(prompt, np.int32)
        out = np.zeros(max(max_new, 1), np.int32)
        n = self.L.uto_greedy_decode(self._h, p, p.size, max_new, out)
        if n < 0:
            raise RuntimeError(f"greedy_decode error {n}")
        return list(prompt) + out[:n].tolist()

    def generate(self, prompt, max_new: int, stop_ids=(), on_token=None) -> list:
        """core::generate, greedy, with stop ids and on_token -> new tokens."""
        p = np.asarray(prompt, np.int32)
        out = np.zeros(max(max_new, 1), np.int32)
        st = np.ascontiguousarray(stop_ids, np.int32)
        cb = TOKEN_FN(lambda _u, t: int(bool(on_token(t)))) if on_token else None
        n = self.L.uto_generate_greedy(self._h, p, p.size, max_new,
                                      st.ctypes.data if st.size else None, st.size,
                                      C.cast(cb, C.c_void_p) if cb else None, None, out)
        if n < 0:
            raise RuntimeError(f"generate error {n}")
        return out[:n].tolist()

    def speculative_loop(self, prompt, max_new: int, depth: int = 1, draft_fn=None,
                         stop_ids=(), on_token=None):
        """speculative_loop (mtp.rs:263-314): draft_fn(tokens, next, depth)
        -> `depth` ids, or None for the native MTP head.
        Returns (tokens, drafted, accepted)."""
        p = np.asarray(prompt, np.int32)
        out = np.zeros(max(max_new, 1), np.int32)
        st = np.ascontiguousarray(stop_ids, np.int32)
        tcb = TOKEN_FN(lambda _u, t: int(bool(on_token(t)))) if on_token else None
        err = []

        def _draft(_u, toks, n, nxt, dep, dst):
            try:
                ids = list(draft_fn([toks[i] for i in range(n)], nxt, dep))
                for i in range(dep):
                    dst[i] = int(ids[i])
                return 0
            except Exception as e:
                err.append(e)
                return -6

        dcb = DRAFT_FN(_draft) if draft_fn else None
        d, a = C.c_int64(), C.c_int64()
        n = self.L.uto_speculative_loop(self._h, p, p.size, max_new, depth,
                                       st.ctypes.data if st.size else None, st.size,
                                       C.cast(tcb, C.c_void_p) if tcb else None, None,
                                       C.cast(dcb, C.c_void_p) if dcb else None, None, out,
                                       C.byref(d), C.byref(a))
        if err:
            raise err[0]
        if n < 0:
            raise RuntimeError(f"speculative_loop error {n}")
        return out[:n].tolist(), d.value, a.value

    def generate_mtp(self, prompt, max_new: int):
        p = np.asarray(prompt, np.int32)
        out = np.zeros(max_new, np.int32)
        d, a = C.c_int64(), C.c_int64()
        n = self.L.uto_generate_mtp(self._h, p, p.size, max_new, out, C.byref(d), C.byref(a))
        if n < 0:
            raise RuntimeError(f"generate_mtp error {n}")
        return out[:n].tolist(), d.value, a.value


class ContextOverflow(RuntimeError):
    pass


class Session:
    def __init__(self, model: Model, path: int = 0):
        self.model = model
        self.L = model.L
        self._h = self.L.uto_session_new(model._h, path)

    def __del__(self):
        if getattr(self, "_mtp", None):
            self.L.uto_mtp_state_free(self._mtp)
            self._mtp = None
        if getattr(self, "_h", None):
            self.L.uto_session_free(self._h)
            self._h = None

    def prefill(self, ids) -> np.ndarray:
        ids = np.asarray(ids, np.int32)
        V = self.model.spec.vocab_size
        out = np.zeros((ids.size, V), np.float32)
        rc = self.L.uto_session_prefill(self._h, ids, ids.size, _vp(out))
        if rc == -2:
            raise ContextOverflow("context overflow")
        if rc != 0:
            raise RuntimeError(f"prefill error {rc}")
        return out

    def decode(self, tok: int) -> np.ndarray:
        return self.prefill([tok])[0]

    def draft_logits(self, next_token: int):
        """draft_logits (mtp.rs:74-133) on this session's MtpState ->
        (logits [vocab], last MTP-layer output row [hidden])."""
        if getattr(self, "_mtp", None) is None:
            self._mtp = self.L.uto_mtp_state_new()
        V, Hd = self.model.spec.vocab_size, self.model.spec.hidden_size
        logits = np.zeros(V, np.float32)
        row = np.zeros(Hd, np.float32)
        rc = self.L.uto_draft_logits(self.model._h, self._h, self._mtp, next_token, logits,
                                    row.ctypes.data)
        if rc != 0:
            raise RuntimeError(f"draft_logits error {rc}")
        return logits, row

    def truncate(self, n: int) -> None:
        self.L.uto_session_truncate(self._h, n)

    @property
    def position(self) -> int:
        return int(self.L.uto_session_position(self._h))
