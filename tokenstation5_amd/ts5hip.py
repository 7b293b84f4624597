"""ctypes binding of libts5hip.so (include/ts5hip.h) for tests and benchmarks.

Everything calls through the C ABI; there is no Python fallback: if the
library is not built, loading raises.
"""
from __future__ import annotations

import ctypes as C
import os
import re
import weakref

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libts5hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "ts5hip.h")

OK, ERR_ARG, ERR_HIP, ERR_UNSUPPORTED, ERR_CONTEXT_FULL, ERR_STATE = 0, -1, -2, -3, -4, -5
F32, F16, Q8_0, Q4_K, Q6_K = 0, 1, 8, 12, 14
KV_F32, KV_F16, KV_Q8 = 0, 1, 2

_vp, _i64, _i32, _u32, _u64, _f32 = C.c_void_p, C.c_int64, C.c_int, C.c_uint32, C.c_uint64, C.c_float


class HParams(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("n_vocab", "n_embd", "n_layer", "n_ff", "n_head", "n_head_kv",
                                          "head_dim", "rope_dims", "rope_neox")] + \
               [(n, C.c_float) for n in ("rms_eps", "rope_base", "attn_scale", "rope_scale", "embd_scale",
                                         "rope_base_swa")] + \
               [(n, C.c_int32) for n in ("gelu", "swa_window", "swa_pattern")]


class CheckResult(C.Structure):
    """ts5hip_check_result: CheckResult (engine/src/checks.h:17-24)."""
    _fields_ = [("n", C.c_int32), ("same_top", C.c_int32), ("worst", C.c_int32), ("max_diff", C.c_double),
                ("rel", C.c_double), ("gpu_ms", C.c_double), ("pass_", C.c_int32), ("saved", C.c_int32)]


class SampleParams(C.Structure):
    """ts5hip_sample_params: SampleParams (engine/src/engine.h:16-23)."""
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_int32), ("max_tokens", C.c_int32),
                ("seed", C.c_uint64), ("draft", C.c_int32), ("adapt", C.c_int32)]


_SIGS = {
    "ts5hip_last_error": (C.c_char_p, [_vp]),
    "ts5hip_init": (_i32, [_i32, C.POINTER(_vp)]),
    "ts5hip_destroy": (None, [_vp]),
    "ts5hip_device_info": (_i32, [_vp, C.POINTER(_i32), C.c_char_p, _i32, C.POINTER(_i64)]),
    "ts5hip_alloc": (_i32, [_vp, C.c_size_t, C.POINTER(_vp)]),
    "ts5hip_free": (_i32, [_vp, _vp]),
    "ts5hip_upload": (_i32, [_vp, _vp, _vp, C.c_size_t]),
    "ts5hip_download": (_i32, [_vp, _vp, _vp, C.c_size_t]),
    "ts5hip_memset": (_i32, [_vp, _vp, _i32, C.c_size_t]),
    "ts5hip_sync": (_i32, [_vp]),
    "ts5hip_timer_begin": (_i32, [_vp]),
    "ts5hip_timer_end": (_i32, [_vp, C.POINTER(_f32)]),
    "ts5hip_timer_mark": (_i32, [_vp, _i32]),
    "ts5hip_timer_marks": (_i32, [_vp, _i32, _vp]),
    "ts5hip_kv_synth": (_i32, [_vp, _u64, _i64, _i32, _vp, _vp]),
    "ts5hip_supports_type": (_i32, [_u32]),
    "ts5hip_weight_bytes": (_i64, [_u32, _i64, _i64]),
    "ts5hip_weight_upload": (_i32, [_vp, _u32, _i64, _i64, _vp, _vp]),
    "ts5hip_weight_synth": (_i32, [_vp, _u32, _i64, _i64, _u64, _i32, _vp]),
    "ts5hip_dequantize": (_i32, [_vp, _u32, _vp, _i64, _i64, _vp]),
    "ts5hip_act_bytes": (_i64, [_i64]),
    "ts5hip_act_quantize": (_i32, [_vp, _vp, _vp, _f32, _i64, _i32, _vp]),
    "ts5hip_rmsnorm": (_i32, [_vp, _vp, _vp, _f32, _i64, _i32, _vp]),
    "ts5hip_matvec": (_i32, [_vp, _u32, _vp, _i64, _i64, _vp, _vp, _f32, _vp, _i32]),
    "ts5hip_matvec_glu": (_i32, [_vp, _u32, _vp, _vp, _i64, _i64, _vp, _vp, _f32, _vp]),
    "ts5hip_matvec_argmax": (_i32, [_vp, _u32, _vp, _i64, _i64, _vp, _vp, _f32, _vp, _vp]),
    "ts5hip_matmul": (_i32, [_vp, C.c_uint32, _vp, C.c_int64, C.c_int64, _vp, _i32, _vp, _f32, _vp, _i32]),
    "ts5hip_matmul_glu": (_i32, [_vp, C.c_uint32, _vp, _vp, C.c_int64, C.c_int64, _vp, _i32, _vp, _f32, _vp]),
    "ts5hip_rope_table": (_i32, [_vp, _i32, _i32, _f32, _f32, _vp, _vp]),
    "ts5hip_rope_kv_append": (_i32, [_vp, _vp, _i32, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _i32, _vp, _vp, _vp,
                                     _f32, _vp, _vp, _vp, _vp, _vp]),
    "ts5hip_attn_decode": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _f32, _i32,
                                  _vp]),
    "ts5hip_attn_decode_f16": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _i32, _vp, _i32, _f32, _i32, _vp]),
    "ts5hip_attn_decode_noalloc": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _i32, _vp, _i32,
                                          _f32, _i32, _vp]),
    "ts5hip_attn_prompt": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _i32, _i32, _f32, _vp]),
    "ts5hip_attn_prompt_f16": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _i32, _i32, _f32, _vp]),
    "ts5hip_argmax": (_i32, [_vp, _vp, _i32, _i32, _vp]),
    "ts5hip_topk": (_i32, [_vp, _vp, _i32, _i32, _vp, _vp]),
    "ts5hip_sampler_new": (_vp, [_u64]),
    "ts5hip_sampler_free": (None, [_vp]),
    "ts5hip_sampler_draw": (C.c_int32, [_vp, _vp, _vp, _i32, _f32, _f32]),
    "ts5hip_model_create": (_i32, [_vp, C.POINTER(HParams), _i32, _i32, C.POINTER(_vp)]),
    "ts5hip_model_destroy": (None, [_vp]),
    "ts5hip_model_set_tensor": (_i32, [_vp, C.c_char_p, _u32, _i64, _i64, _vp]),
    "ts5hip_model_synth_tensor": (_i32, [_vp, C.c_char_p, _u32, _i64, _i64, _u64, _i32]),
    "ts5hip_forward": (_i32, [_vp, _vp, _i32, _i32, _vp, _i32]),
    "ts5hip_forward_in_place": (_i32, [_vp, _vp, _i32, _i32, _i32]),
    "ts5hip_logits_view": (C.POINTER(C.c_float), [_vp]),
    "ts5hip_n_ctx": (_i32, [_vp]),
    "ts5hip_kv_type": (_i32, [_vp]),
    "ts5hip_token_path": (_i32, [_vp]),
    "ts5hip_model_sample": (C.c_int32, [_vp, _vp, _i32, _f32, _f32, _i32]),
    "ts5hip_logits_topk": (_i32, [_vp, _i32, _i32, _i32, _vp, _vp]),
    "ts5hip_generate_greedy": (_i32, [_vp, C.c_int32, _i32, _i32, _vp]),
    "ts5hip_kv_read": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp]),
    "ts5hip_kv_write": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp]),
    "ts5hip_take_profile": (_i32, [_vp, C.c_char_p, _i32]),
    "ts5hip_model_set_tensor_rows": (_i32, [_vp, C.c_char_p, _u32, _i64, _i64, _i64, _i64, _vp]),
    "ts5hip_kv_bytes_per_token": (_u64, [C.POINTER(HParams), _i32]),
    "ts5hip_fit_context": (_i32, [_u64, _u64, _u64, _i32]),
    "ts5hip_f16_reaches": (_i32, [_i32, _i32]),
    "ts5hip_gguf_hparams": (_i32, [C.c_char_p, C.POINTER(HParams), C.POINTER(_i32), C.POINTER(_i64)]),
    "ts5hip_model_load": (_i32, [_vp, C.c_char_p, _i32, _i32, _i32, C.POINTER(_vp), C.POINTER(_i32)]),
    "ts5hip_check_tokens": (_i32, [_i32, _i32, _vp]),
    "ts5hip_model_file_id": (_i32, [C.c_char_p, C.POINTER(_u64), C.POINTER(_u64)]),
    "ts5hip_ref_path": (_i32, [C.c_char_p, _i32, C.c_char_p, _i32]),
    "ts5hip_ref_load": (_i32, [C.c_char_p, _i32, _i32, _i32, _vp]),
    "ts5hip_ref_save": (_i32, [C.c_char_p, _i32, _i32, _i32, _vp]),
    "ts5hip_check_run": (_i32, [_vp, C.c_char_p, _i32, _vp, _vp]),
    "ts5hip_engine_new": (_i32, [_vp, C.POINTER(_vp)]),
    "ts5hip_engine_free": (None, [_vp]),
    "ts5hip_engine_set_drafter": (_i32, [_vp, _vp]),
    "ts5hip_engine_generate": (_i32, [_vp, _vp, _i32, C.POINTER(SampleParams), _vp, _i32, _vp, _vp]),
    "ts5hip_engine_drafter_state": (_i32, [_vp]),
    "ts5hip_engine_draft_sources": (_i32, [_vp, _vp]),
}

_lib = None


def header_symbols() -> list[str]:
    """Every function include/ts5hip.h declares."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(ts5hip_[a-z0-9_]+)\s*\(", text)))


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build() (no CPU fallback exists)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


class Ts5HipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"ts5hip error {code}: {msg}")
        self.code = code


def _ptr(a) -> int | None:
    if a is None:
        return None
    if isinstance(a, DeviceBuffer):
        return a.ptr
    if isinstance(a, np.ndarray):
        assert a.flags["C_CONTIGUOUS"]
        return a.ctypes.data
    return int(a)


class DeviceBuffer:
    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx, self.nbytes = ctx, int(nbytes)
        p = _vp()
        ctx.check(lib().ts5hip_alloc(ctx.h, self.nbytes, C.byref(p)))
        self.ptr = p.value

    def free(self):
        if self.ptr:
            self.ctx.check(lib().ts5hip_free(self.ctx.h, self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and self.ctx.h:
                lib().ts5hip_free(self.ctx.h, self.ptr)
        except Exception:
            pass

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes, (a.nbytes, self.nbytes)
        self.ctx.check(lib().ts5hip_upload(self.ctx.h, self.ptr, a.ctypes.data, a.nbytes))
        return self

    def download(self, dtype, shape=None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        count = (self.nbytes - offset) // dtype.itemsize if shape is None else int(np.prod(shape))
        out = np.empty(count, dtype)
        self.ctx.check(lib().ts5hip_download(self.ctx.h, out.ctypes.data, self.ptr + offset, out.nbytes))
        return out if shape is None else out.reshape(shape)

    def zero(self):
        self.ctx.check(lib().ts5hip_memset(self.ctx.h, self.ptr, 0, self.nbytes))
        return self


class Context:
    def __init__(self, device: int = 0):
        self.h = None
        self._models = weakref.WeakSet()  # destroyed before the context
        h = _vp()
        rc = lib().ts5hip_init(device, C.byref(h))
        if rc != OK:
            raise Ts5HipError(rc, lib().ts5hip_last_error(None).decode())
        self.h = h.value
        n_cu, hbm = _i32(), _i64()
        arch = C.create_string_buffer(64)
        self.check(lib().ts5hip_device_info(self.h, C.byref(n_cu), arch, 64, C.byref(hbm)))
        self.n_cu, self.arch, self.hbm = n_cu.value, arch.value.decode(), hbm.value

    def close(self):
        if self.h:
            for m in list(self._models):
                m.close()
            lib().ts5hip_destroy(self.h)
            self.h = None

    def check(self, rc: int):
        if rc != OK:
            raise Ts5HipError(rc, lib().ts5hip_last_error(self.h).decode())
        return rc

    # -- memory ------------------------------------------------------------------
    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def to_device(self, a: np.ndarray) -> DeviceBuffer:
        a = np.ascontiguousarray(a)
        return DeviceBuffer(self, max(a.nbytes, 1)).upload(a)

    def sync(self):
        self.check(lib().ts5hip_sync(self.h))

    def timer_begin(self):
        self.check(lib().ts5hip_timer_begin(self.h))

    def timer_end(self) -> float:
        ms = _f32()
        self.check(lib().ts5hip_timer_end(self.h, C.byref(ms)))
        return ms.value

    # -- weights -----------------------------------------------------------------
    @staticmethod
    def weight_bytes(t: int, ne0: int, ne1: int) -> int:
        return lib().ts5hip_weight_bytes(t, ne0, ne1)

    def weight(self, t: int, ne0: int, ne1: int, gguf: np.ndarray) -> DeviceBuffer:
        """GGUF bytes (ne1, row_bytes) uint8 -> a device buffer in HBM layout."""
        n = self.weight_bytes(t, ne0, ne1)
        if n < 0:
            raise Ts5HipError(ERR_UNSUPPORTED, f"type {t} {ne1}x{ne0}")
        d = DeviceBuffer(self, n)
        g = np.ascontiguousarray(gguf, np.uint8)
        self.check(lib().ts5hip_weight_upload(self.h, t, ne0, ne1, g.ctypes.data, d.ptr))
        return d

    def timer_mark(self, i: int):
        self.check(lib().ts5hip_timer_mark(self.h, i))

    def timer_marks(self, n: int) -> np.ndarray:
        """The n - 1 intervals (ms) between marks 0..n-1."""
        out = np.empty(n - 1, np.float32)
        self.check(lib().ts5hip_timer_marks(self.h, n, out.ctypes.data))
        return out

    def kv_synth(self, seed: int, n: int, kv: int, values, scales=None):
        """n N(0,1) values into a q8 (values + scales) or f16 cache layout."""
        self.check(lib().ts5hip_kv_synth(self.h, seed, n, kv, _ptr(values), _ptr(scales) if scales is not None else None))

    def weight_synth(self, t: int, ne0: int, ne1: int, seed: int, centered: bool = False) -> DeviceBuffer:
        d = DeviceBuffer(self, self.weight_bytes(t, ne0, ne1))
        self.check(lib().ts5hip_weight_synth(self.h, t, ne0, ne1, seed, int(centered), d.ptr))
        return d

    # -- ops (device buffers in and out) --------------------------------------------
    def dequantize(self, t, w, ne0, rows, y):
        self.check(lib().ts5hip_dequantize(self.h, t, _ptr(w), ne0, rows, _ptr(y)))

    @staticmethod
    def act_bytes(n: int) -> int:
        return lib().ts5hip_act_bytes(n)

    def act_quantize(self, x, norm_w, eps, n, ntok, act):
        self.check(lib().ts5hip_act_quantize(self.h, _ptr(x), _ptr(norm_w), eps, n, ntok, _ptr(act)))

    def rmsnorm(self, x, w, eps, n, ntok, y):
        self.check(lib().ts5hip_rmsnorm(self.h, _ptr(x), _ptr(w), eps, n, ntok, _ptr(y)))

    def matmul(self, t, w, ne0, ne1, x, ntok, y, norm_w=None, eps=0.0, accumulate=False):
        self.check(lib().ts5hip_matmul(self.h, t, _ptr(w), ne0, ne1, _ptr(x), ntok, _ptr(norm_w), eps, _ptr(y),
                                       int(accumulate)))

    def matmul_glu(self, t, wg, wu, ne0, ne1, x, ntok, y, norm_w=None, eps=0.0):
        self.check(lib().ts5hip_matmul_glu(self.h, t, _ptr(wg), _ptr(wu), ne0, ne1, _ptr(x), ntok, _ptr(norm_w), eps,
                                           _ptr(y)))

    def matvec(self, t, w, ne0, ne1, x, y, norm_w=None, eps=0.0, accumulate=False):
        self.check(lib().ts5hip_matvec(self.h, t, _ptr(w), ne0, ne1, _ptr(x), _ptr(norm_w), eps, _ptr(y),
                                       int(accumulate)))

    def matvec_glu(self, t, wg, wu, ne0, ne1, x, y, norm_w=None, eps=0.0):
        self.check(lib().ts5hip_matvec_glu(self.h, t, _ptr(wg), _ptr(wu), ne0, ne1, _ptr(x), _ptr(norm_w), eps,
                                           _ptr(y)))

    def matvec_argmax(self, t, w, ne0, ne1, x, y, out, norm_w=None, eps=0.0):
        self.check(lib().ts5hip_matvec_argmax(self.h, t, _ptr(w), ne0, ne1, _ptr(x), _ptr(norm_w), eps, _ptr(y),
                                              _ptr(out)))

    def rope_table(self, n_rot, n_pos, base, scale=1.0, freqs=None) -> DeviceBuffer:
        d = DeviceBuffer(self, n_pos * n_rot * 4)
        f = None if freqs is None else np.ascontiguousarray(freqs, np.float32)
        self.check(lib().ts5hip_rope_table(self.h, n_rot, n_pos, base, scale, _ptr(f), d.ptr))
        return d

    def rope_kv_append(self, qkv, ntok, pos0_dev, H, HKV, HD, n_rot, neox, rope_cs, n_ctx, q_out, k8, ks, v8, vs,
                       bias=None, q_norm=None, k_norm=None, eps=1e-6):
        self.check(lib().ts5hip_rope_kv_append(self.h, _ptr(qkv), ntok, _ptr(pos0_dev), H, HKV, HD, n_rot, int(neox),
                                               _ptr(rope_cs), n_ctx, _ptr(bias), _ptr(q_norm), _ptr(k_norm), eps,
                                               _ptr(q_out), _ptr(k8), _ptr(ks), _ptr(v8), _ptr(vs)))

    def attn_decode(self, q, B, H, HKV, HD, k8, ks, v8, vs, n_ctx, n_keys_dev, kv_per_batch, scale, out,
                    n_split=0):
        self.check(lib().ts5hip_attn_decode(self.h, _ptr(q), B, H, HKV, HD, _ptr(k8), _ptr(ks), _ptr(v8), _ptr(vs),
                                            n_ctx, _ptr(n_keys_dev), int(kv_per_batch), scale, n_split, _ptr(out)))

    def attn_decode_f16(self, q, B, H, HKV, HD, k16, v16, n_ctx, n_keys_dev, kv_per_batch, scale, out, n_split=0):
        self.check(lib().ts5hip_attn_decode_f16(self.h, _ptr(q), B, H, HKV, HD, _ptr(k16), _ptr(v16), n_ctx,
                                                _ptr(n_keys_dev), int(kv_per_batch), scale, n_split, _ptr(out)))

    def attn_decode_noalloc(self, q, B, H, HKV, HD, k8, ks, v8, vs, n_ctx, n_keys_dev, kv_per_batch, scale, out,
                            n_split=0):
        self.check(lib().ts5hip_attn_decode_noalloc(self.h, _ptr(q), B, H, HKV, HD, _ptr(k8), _ptr(ks), _ptr(v8),
                                                    _ptr(vs), n_ctx, _ptr(n_keys_dev), int(kv_per_batch), scale,
                                                    n_split, _ptr(out)))

    def attn_prompt(self, q, nq, H, HKV, HD, k8, ks, v8, vs, n_ctx, pos0, scale, out):
        self.check(lib().ts5hip_attn_prompt(self.h, _ptr(q), nq, H, HKV, HD, _ptr(k8), _ptr(ks), _ptr(v8), _ptr(vs),
                                            n_ctx, pos0, scale, _ptr(out)))


    def attn_prompt_f16(self, q, nq, H, HKV, HD, k16, v16, n_ctx, pos0, scale, out):
        self.check(lib().ts5hip_attn_prompt_f16(self.h, _ptr(q), nq, H, HKV, HD, _ptr(k16), _ptr(v16), n_ctx, pos0,
                                                scale, _ptr(out)))
    def argmax(self, x, n, rows, out):
        self.check(lib().ts5hip_argmax(self.h, _ptr(x), n, rows, _ptr(out)))

    def topk(self, x, n, k, vals, ids):
        self.check(lib().ts5hip_topk(self.h, _ptr(x), n, k, _ptr(vals), _ptr(ids)))


class Sampler:
    def __init__(self, seed: int):
        self.h = lib().ts5hip_sampler_new(seed)

    def __del__(self):
        if getattr(self, "h", None):
            lib().ts5hip_sampler_free(self.h)
            self.h = None

    def draw(self, ids, logits, temperature, top_p) -> int:
        ids = np.ascontiguousarray(ids, np.int32)
        lg = np.ascontiguousarray(logits, np.float32)
        return int(lib().ts5hip_sampler_draw(self.h, ids.ctypes.data, lg.ctypes.data, ids.size, temperature, top_p))


def hparams(hp: dict) -> HParams:
    """HParams of a synth.py model dict (engine/src/model.cpp:13-68 derivations)."""
    f32 = np.float32
    h = HParams(n_vocab=hp["n_vocab"], n_embd=hp["n_embd"], n_layer=hp["n_layer"], n_ff=hp["n_ff"],
                n_head=hp["n_head"], n_head_kv=hp["n_head_kv"], head_dim=hp["head_dim"],
                rope_dims=hp.get("rope_dims", hp["head_dim"]),
                rope_neox=int(hp["arch"] in ("qwen2", "qwen3", "gemma3")),
                rms_eps=hp["rms_eps"], rope_base=hp["rope_base"],
                attn_scale=float(f32(1.0) / np.sqrt(f32(hp["head_dim"]))), rope_scale=1.0)
    if hp["arch"] == "gemma3":  # model.cpp:44-63
        h.embd_scale = float(np.sqrt(f32(hp["n_embd"])))
        h.gelu, h.swa_window, h.swa_pattern, h.rope_base_swa = 1, hp.get("swa_window", 0), 6, 10000.0
        if hp.get("rope_scaling_factor"):  # linear scaling (model.cpp:53-56)
            h.rope_scale = float(np.float32(1.0 / hp["rope_scaling_factor"]))
        if hp["n_layer"] == 62:
            h.attn_scale = float(f32(1.0) / np.sqrt(f32(hp["n_embd"] // hp["n_head"])))
    return h


class Model:
    """Backend (engine/src/backend.h:16-44) over libts5hip.so."""

    def __init__(self, ctx: Context, hp: dict, n_ctx: int, kv: int = KV_Q8):
        self.ctx, self.hp, self.h = ctx, hp, None
        self._hp = hparams(hp)
        h = _vp()
        ctx.check(lib().ts5hip_model_create(ctx.h, C.byref(self._hp), n_ctx, kv, C.byref(h)))
        self.h = h.value
        ctx._models.add(self)
        self.n_vocab = hp["n_vocab"]

    def close(self):
        # A model lives inside its context: after the context is gone there is
        # nothing left to free (ts5hip_destroy must not precede model_destroy).
        if self.h and self.ctx.h:
            lib().ts5hip_model_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_tensors(self, tensors: dict):
        """{name: (type, ne0, ne1, gguf uint8 array)} (synth.model_tensors)."""
        for name, (t, ne0, ne1, data) in tensors.items():
            d = np.ascontiguousarray(data, np.uint8)
            self.ctx.check(lib().ts5hip_model_set_tensor(self.h, name.encode(), t, ne0, ne1, d.ctypes.data))

    def synth_tensor(self, name: str, t: int, ne0: int, ne1: int, seed: int, centered: bool = False):
        self.ctx.check(lib().ts5hip_model_synth_tensor(self.h, name.encode(), t, ne0, ne1, seed, int(centered)))

    def forward(self, tokens, pos0: int, logits: bool = True, all_logits: bool = False):
        tok = np.ascontiguousarray(tokens, np.int32)
        n = tok.size
        out = np.empty(((n if all_logits else 1), self.n_vocab), np.float32) if logits else None
        self.ctx.check(lib().ts5hip_forward(self.h, tok.ctypes.data, n, pos0, _ptr(out), int(all_logits)))
        return out

    def forward_in_place(self, tokens, pos0: int, all_logits: bool = False) -> np.ndarray:
        tok = np.ascontiguousarray(tokens, np.int32)
        self.ctx.check(lib().ts5hip_forward_in_place(self.h, tok.ctypes.data, tok.size, pos0, int(all_logits)))
        rows = tok.size if all_logits else 1
        p = lib().ts5hip_logits_view(self.h)
        return np.ctypeslib.as_array(p, shape=(rows, self.n_vocab))

    def sample(self, sampler: Sampler, row: int, temperature: float, top_p: float, top_k: int) -> int:
        r = lib().ts5hip_model_sample(self.h, sampler.h, row, temperature, top_p, top_k)
        if r < 0:
            self.ctx.check(r)
        return int(r)

    def logits_topk(self, row0: int, nrows: int, k: int):
        """The k largest logits of rows row0.. of the last forward, found on the GPU: (vals, ids) [nrows][k]."""
        v = np.empty((nrows, k), np.float32)
        i = np.empty((nrows, k), np.int32)
        self.ctx.check(lib().ts5hip_logits_topk(self.h, row0, nrows, k, v.ctypes.data, i.ctypes.data))
        return v, i

    def generate_greedy(self, token: int, pos: int, n_steps: int) -> np.ndarray:
        out = np.empty(n_steps, np.int32)
        self.ctx.check(lib().ts5hip_generate_greedy(self.h, token, pos, n_steps, out.ctypes.data))
        return out

    def n_ctx(self) -> int:
        return lib().ts5hip_n_ctx(self.h)

    def check_run(self, model_path: "str | None", n: int, ref_logits: "np.ndarray | None" = None) -> CheckResult:
        """ts5 check (run_check) of this model against ref_logits or the saved .ts5ref of model_path."""
        r = CheckResult()
        ref = None if ref_logits is None else np.ascontiguousarray(ref_logits, np.float32)
        self.ctx.check(lib().ts5hip_check_run(self.h, model_path.encode() if model_path else None, n,
                                              _ptr(ref), C.byref(r)))
        return r

    def kv_write(self, layer: int, which: int, pos0: int, values: np.ndarray):
        """fp32 [n][n_head_kv * head_dim] into the cache at pos0.., rounded as the cache keeps them."""
        v = np.ascontiguousarray(values, np.float32)
        self.ctx.check(lib().ts5hip_kv_write(self.h, layer, which, pos0, v.shape[0], v.ctypes.data))

    def kv_type(self) -> int:
        return lib().ts5hip_kv_type(self.h)

    def kv(self, layer: int, which: int, pos0: int, n: int) -> np.ndarray:
        w = self.hp["n_head_kv"] * self.hp["head_dim"]
        out = np.empty((n, w), np.float32)
        self.ctx.check(lib().ts5hip_kv_read(self.h, layer, which, pos0, n, out.ctypes.data))
        return out

    def token_path(self) -> str:
        """How single-token steps run: "graphs" or "direct"."""
        rc = lib().ts5hip_token_path(self.h)
        self.ctx.check(min(rc, 0))
        return ("direct", "graphs")[rc]

    def take_profile(self) -> str:
        """Backend::take_profile: the profile text since the last call (empty unless TS5_PROFILE was set)."""
        buf = C.create_string_buffer(1 << 16)
        self.ctx.check(lib().ts5hip_take_profile(self.h, buf, 1 << 16))
        return buf.value.decode()


def load_model(ctx: "Context", path: str, n_ctx: int = 0, kv: int = KV_Q8, threads: int = 0) -> "Model":
    """ts5hip_model_load: a Model of a GGUF file (n_ctx 0: the context that fits)."""
    h, kv_out = _vp(), _i32()
    ctx.check(lib().ts5hip_model_load(ctx.h, path.encode(), n_ctx, kv, threads, C.byref(h), C.byref(kv_out)))
    hp_raw, _, _ = gguf_hparams(path)
    m = Model.__new__(Model)
    m.ctx, m.hp, m.h = ctx, hp_raw, h.value
    ctx._models.add(m)
    m.n_vocab = hp_raw["n_vocab"]
    m.chosen_kv = kv_out.value
    return m


class Engine:
    """Engine (engine/src/engine.h:33-66): generation with prompt-lookup and
    draft-model speculation over a Model."""

    def __init__(self, model: Model):
        self.model = model
        h = _vp()
        model.ctx.check(lib().ts5hip_engine_new(model.h, C.byref(h)))
        self.h = h.value

    def set_drafter(self, dm: "Model | None"):
        self.drafter = dm
        self.model.ctx.check(lib().ts5hip_engine_set_drafter(self.h, dm.h if dm else None))

    def generate(self, prompt, temperature=0.0, top_p=0.95, top_k=40, max_tokens=64, seed=0, draft=-1, adapt=True,
                 eog=()):
        """(ids, stats): stats = prompt, evaluated, generated, drafted, accepted, stopped."""
        prompt = np.ascontiguousarray(prompt, np.int32)
        eog = np.ascontiguousarray(eog, np.int32)
        out = np.empty(max(max_tokens, 1), np.int32)
        stats = np.zeros(6, np.int32)
        p = SampleParams(temperature, top_p, top_k, max_tokens, seed, draft, int(adapt))
        n = lib().ts5hip_engine_generate(self.h, prompt.ctypes.data, prompt.size, C.byref(p),
                                         eog.ctypes.data if eog.size else None, eog.size, out.ctypes.data,
                                         stats.ctypes.data)
        self.model.ctx.check(min(n, 0))
        return out[:n], stats

    def draft_sources(self) -> dict:
        """The last generation's drafts by source: lookup / model, drafted and accepted."""
        out = np.zeros(4, np.int32)
        self.model.ctx.check(lib().ts5hip_engine_draft_sources(self.h, out.ctypes.data))
        return dict(lookup_drafted=int(out[0]), lookup_accepted=int(out[1]), model_drafted=int(out[2]),
                    model_accepted=int(out[3]))

    def drafter_state(self) -> int:
        """0 no draft model, 1 drafting, 2 stopped (Engine::drafter_ok_ false)."""
        return int(lib().ts5hip_engine_drafter_state(self.h))

    def close(self):
        if self.h:
            lib().ts5hip_engine_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- GGUF files, KV sizing, ts5 check --------------------------------------------------------

def kv_bytes_per_token(hp: dict, kv: int) -> int:
    h = hparams(hp)
    return int(lib().ts5hip_kv_bytes_per_token(C.byref(h), kv))


def fit_context(memory: int, used: int, per_token: int, cap: int) -> int:
    return int(lib().ts5hip_fit_context(memory, used, per_token, cap))


def f16_reaches(f16_ctx: int, train: int) -> bool:
    return bool(lib().ts5hip_f16_reaches(f16_ctx, train))


def gguf_hparams(path: str):
    """(hparams fields as a dict, training context, HBM bytes beside the KV cache) of a GGUF file."""
    h, train, fixed = HParams(), _i32(), _i64()
    rc = lib().ts5hip_gguf_hparams(path.encode(), C.byref(h), C.byref(train), C.byref(fixed))
    if rc != OK:
        raise Ts5HipError(rc, lib().ts5hip_last_error(None).decode())
    return {f: getattr(h, f) for f, _ in HParams._fields_}, train.value, fixed.value


def check_tokens(n: int, n_vocab: int) -> np.ndarray:
    out = np.empty(n, np.int32)
    rc = lib().ts5hip_check_tokens(n, n_vocab, out.ctypes.data)
    if rc != OK:
        raise Ts5HipError(rc, lib().ts5hip_last_error(None).decode())
    return out


def model_file_id(path: str):
    size, h = _u64(), _u64()
    rc = lib().ts5hip_model_file_id(path.encode(), C.byref(size), C.byref(h))
    if rc != OK:
        raise Ts5HipError(rc, lib().ts5hip_last_error(None).decode())
    return size.value, h.value


def ref_path(model_path: str, kv: int) -> str:
    buf = C.create_string_buffer(4096)
    rc = lib().ts5hip_ref_path(model_path.encode(), kv, buf, 4096)
    if rc != OK:
        raise Ts5HipError(rc, lib().ts5hip_last_error(None).decode())
    return buf.value.decode()


def ref_load(model_path: str, n: int, n_vocab: int, kv: int) -> np.ndarray:
    out = np.empty((n, n_vocab), np.float32)
    rc = lib().ts5hip_ref_load(model_path.encode(), n, n_vocab, kv, out.ctypes.data)
    if rc != OK:
        raise Ts5HipError(rc, lib().ts5hip_last_error(None).decode())
    return out


def ref_save(model_path: str, kv: int, logits: np.ndarray) -> None:
    lg = np.ascontiguousarray(logits, np.float32)
    rc = lib().ts5hip_ref_save(model_path.encode(), lg.shape[0], lg.shape[1], kv, lg.ctypes.data)
    if rc != OK:
        raise Ts5HipError(rc, lib().ts5hip_last_error(None).decode())
