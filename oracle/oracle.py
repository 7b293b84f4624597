"""TEST INFRASTRUCTURE ONLY: ctypes access to the CPU oracle (libts5oracle.so)
and, where it was built, to ts5's own CPU code (_ref/libts5ref.so).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module. The oracle is the checker, never the thing measured or shipped.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libts5oracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libts5ref.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


class HParams(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("n_vocab", "n_embd", "n_layer", "n_ff", "n_head", "n_head_kv",
                                          "head_dim", "rope_dims", "rope_neox")] + \
               [(n, C.c_float) for n in ("rms_eps", "rope_base", "attn_scale", "rope_scale", "embd_scale",
                                         "rope_base_swa")] + \
               [(n, C.c_int32) for n in ("gelu", "swa_window", "swa_pattern")]


class Tensor(C.Structure):
    _fields_ = [("type", C.c_uint32), ("ne0", C.c_int64), ("ne1", C.c_int64), ("data", C.c_void_p)]


class Layer(C.Structure):
    _fields_ = [(n, Tensor) for n in ("attn_norm", "wq", "wk", "wv", "wo", "bq", "bk", "bv", "q_norm", "k_norm",
                                      "ffn_norm", "w_gate", "w_up", "w_down", "post_attn_norm", "post_ffn_norm")]


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = C.CDLL(LIB)
        L.ts5o_fp16_to_fp32.restype = C.c_float
        L.ts5o_fp16_to_fp32.argtypes = [C.c_uint16]
        L.ts5o_fp32_to_fp16.restype = C.c_uint16
        L.ts5o_fp32_to_fp16.argtypes = [C.c_float]
        L.ts5o_dequantize_row.argtypes = [C.c_uint32, C.c_void_p, _f32p, C.c_int64]
        L.ts5o_matmul.argtypes = [C.c_uint32, C.c_void_p, C.c_int64, C.c_int64, C.c_int64, _f32p, C.c_int,
                                  _f32p, C.c_int64, C.c_int]
        L.ts5o_rmsnorm.argtypes = [_f32p, _f32p, C.c_int, C.c_float]
        L.ts5o_rope.argtypes = [_f32p, C.c_int, C.c_int, C.c_float, C.c_int, C.c_void_p, C.c_float]
        L.ts5o_rope_cs.argtypes = [C.c_int, C.c_int, C.c_float, C.c_void_p, C.c_float, _f32p, _f32p]
        L.ts5o_round_kv.argtypes = [C.c_int, _f32p, C.c_int]
        L.ts5o_attention.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                                     _f32p]
        L.ts5o_swiglu.argtypes = [_f32p, _f32p, C.c_int64]
        L.ts5o_geglu.argtypes = [_f32p, _f32p, C.c_int64]
        L.ts5o_sampler_new.restype = C.c_void_p
        L.ts5o_sampler_new.argtypes = [C.c_uint64]
        L.ts5o_sampler_free.argtypes = [C.c_void_p]
        L.ts5o_sample.restype = C.c_int32
        L.ts5o_sample.argtypes = [C.c_void_p, _f32p, C.c_int, C.c_float, C.c_float, C.c_int]
        L.ts5o_sample_topk.restype = C.c_int32
        L.ts5o_sample_topk.argtypes = [C.c_void_p, _i32p, _f32p, C.c_int, C.c_float, C.c_float]
        L.ts5o_model_new.restype = C.c_void_p
        L.ts5o_model_new.argtypes = [C.POINTER(HParams), C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor),
                                     C.POINTER(Tensor), C.POINTER(Layer), C.c_int, C.c_int, C.c_int]
        L.ts5o_model_free.argtypes = [C.c_void_p]
        L.ts5o_forward.argtypes = [C.c_void_p, _i32p, C.c_int, C.c_int, C.c_void_p, C.c_int]
        L.ts5o_kv.restype = C.POINTER(C.c_float)
        L.ts5o_kv.argtypes = [C.c_void_p, C.c_int, C.c_int]
        _lib = L
    return _lib


# --- elementwise helpers --------------------------------------------------------

def dequantize(t: int, raw: np.ndarray, n: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(n, np.float32)
    if lib().ts5o_dequantize_row(t, raw.ctypes.data, out, n) != 0:
        raise ValueError(f"unsupported type {t}")
    return out


def matmul(t: int, w: np.ndarray, ne0: int, x: np.ndarray, threads: int = 0) -> np.ndarray:
    """w: (rows, row_bytes) uint8; x: (n, ne0) fp32 -> (n, rows) fp32."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    rows = w.shape[0]
    y = np.empty((x.shape[0], rows), np.float32)
    lib().ts5o_matmul(t, w.ctypes.data, w.shape[1], ne0, rows, x, x.shape[0], y, rows, threads)
    return y


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.array(x, np.float32)
    lib().ts5o_rmsnorm(x, np.ascontiguousarray(w, np.float32), x.size, eps)
    return x


def round_kv(kv: int, v: np.ndarray) -> np.ndarray:
    v = np.array(v, np.float32)
    lib().ts5o_round_kv(kv, v, v.size)
    return v


def rope_cs(n_rot: int, pos: int, base: float, scale: float = 1.0):
    c = np.empty(n_rot // 2, np.float32)
    s = np.empty(n_rot // 2, np.float32)
    lib().ts5o_rope_cs(n_rot, pos, base, None, scale, c, s)
    return c, s


def rope(v: np.ndarray, n_rot: int, pos: int, base: float, neox: bool, scale: float = 1.0) -> np.ndarray:
    v = np.array(v, np.float32)
    lib().ts5o_rope(v, n_rot, pos, base, int(neox), None, scale)
    return v


def attention(q, kc, vc, H, HKV, HD, pos, scale, lo=0):
    q = np.ascontiguousarray(q, np.float32)
    out = np.empty(H * HD, np.float32)
    lib().ts5o_attention(q, np.ascontiguousarray(kc, np.float32), np.ascontiguousarray(vc, np.float32), H, HKV,
                         HD, lo, pos, scale, out)
    return out


def swiglu(g, u):
    g = np.array(g, np.float32)
    lib().ts5o_swiglu(g, np.ascontiguousarray(u, np.float32), g.size)
    return g


def geglu(g, u):
    g = np.array(g, np.float32)
    lib().ts5o_geglu(g, np.ascontiguousarray(u, np.float32), g.size)
    return g


class Sampler:
    def __init__(self, seed: int):
        self.h = lib().ts5o_sampler_new(seed)

    def __del__(self):
        if getattr(self, "h", None):
            lib().ts5o_sampler_free(self.h)

    def sample(self, logits, temperature, top_p, top_k) -> int:
        lg = np.ascontiguousarray(logits, np.float32)
        return int(lib().ts5o_sample(self.h, lg, lg.size, temperature, top_p, top_k))

    def sample_topk(self, ids, logits, temperature, top_p) -> int:
        ids = np.ascontiguousarray(ids, np.int32)
        lg = np.ascontiguousarray(logits, np.float32)
        return int(lib().ts5o_sample_topk(self.h, ids, lg, ids.size, temperature, top_p))


# --- whole model ------------------------------------------------------------------

def hparams(hp: dict) -> HParams:
    """Model::open's derived values (engine/src/model.cpp:36-63) for a synth.py dict."""
    f32 = np.float32
    h = HParams(n_vocab=hp["n_vocab"], n_embd=hp["n_embd"], n_layer=hp["n_layer"], n_ff=hp["n_ff"],
                n_head=hp["n_head"], n_head_kv=hp["n_head_kv"], head_dim=hp["head_dim"],
                rope_dims=hp.get("rope_dims", hp["head_dim"]),
                rope_neox=int(hp["arch"] in ("qwen2", "qwen3", "gemma3")),
                rms_eps=hp["rms_eps"], rope_base=hp["rope_base"],
                attn_scale=float(f32(1.0) / np.sqrt(f32(hp["head_dim"]))),
                rope_scale=1.0)
    if hp["arch"] == "gemma3":
        h.embd_scale = float(np.sqrt(f32(hp["n_embd"])))
        h.gelu = 1
        h.swa_window = hp.get("swa_window", 0)
        h.swa_pattern = 6
        h.rope_base_swa = 10000.0
        if hp.get("rope_scaling_factor"):  # linear scaling (model.cpp:53-56)
            h.rope_scale = float(np.float32(1.0 / hp["rope_scaling_factor"]))
        if hp["n_layer"] == 62:
            h.attn_scale = float(f32(1.0) / np.sqrt(f32(hp["n_embd"] // hp["n_head"])))
    return h


class Model:
    """CpuBackend restated over tensors held in numpy arrays (synth.model_tensors)."""

    def __init__(self, hp: dict, tensors: dict, n_ctx: int, kv: int, threads: int = 0):
        self.hp, self.tensors = hp, tensors
        self._keep = []

        def T(name):
            if name not in tensors:
                return Tensor(0, 0, 0, None)
            t, ne0, ne1, data = tensors[name]
            data = np.ascontiguousarray(data)
            self._keep.append(data)
            return Tensor(t, ne0, ne1, data.ctypes.data)

        layers = (Layer * hp["n_layer"])()
        for i in range(hp["n_layer"]):
            p = f"blk.{i}."
            layers[i] = Layer(T(p + "attn_norm.weight"), T(p + "attn_q.weight"), T(p + "attn_k.weight"),
                              T(p + "attn_v.weight"), T(p + "attn_output.weight"), T(p + "attn_q.bias"),
                              T(p + "attn_k.bias"), T(p + "attn_v.bias"), T(p + "attn_q_norm.weight"),
                              T(p + "attn_k_norm.weight"), T(p + "ffn_norm.weight"), T(p + "ffn_gate.weight"),
                              T(p + "ffn_up.weight"), T(p + "ffn_down.weight"), T(p + "post_attention_norm.weight"),
                              T(p + "post_ffw_norm.weight"))
        self._hp = hparams(hp)
        emb, onorm, out, freqs = T("token_embd.weight"), T("output_norm.weight"), T("output.weight"), \
            T("rope_freqs.weight")
        self.h = lib().ts5o_model_new(C.byref(self._hp), C.byref(emb), C.byref(onorm), C.byref(out),
                                      C.byref(freqs) if freqs.data else None, layers, n_ctx, kv, threads)
        self.n_ctx = n_ctx

    def __del__(self):
        if getattr(self, "h", None):
            lib().ts5o_model_free(self.h)

    def forward(self, tokens, pos0: int, logits: bool = True, all_logits: bool = False):
        tok = np.ascontiguousarray(tokens, np.int32)
        n = tok.size
        out = np.empty(((n if all_logits else 1), self.hp["n_vocab"]), np.float32) if logits else None
        rc = lib().ts5o_forward(self.h, tok, n, pos0, out.ctypes.data if logits else None, int(all_logits))
        if rc != 0:
            raise RuntimeError("context full")
        return out

    def kv(self, which: int, layer: int) -> np.ndarray:
        kvw = self.hp["n_head_kv"] * self.hp["head_dim"]
        p = lib().ts5o_kv(self.h, which, layer)
        return np.ctypeslib.as_array(p, shape=(self.n_ctx, kvw))


# --- the reference's own CPU code (built only where its sources are present) --------

_ref = None


def ref_available() -> bool:
    return os.path.exists(REF_LIB)


def ref():
    global _ref
    if _ref is None:
        L = C.CDLL(REF_LIB)
        L.ts5r_last_error.restype = C.c_char_p
        L.ts5r_fp16_to_fp32.restype = C.c_float
        L.ts5r_fp16_to_fp32.argtypes = [C.c_uint16]
        L.ts5r_fp32_to_fp16.restype = C.c_uint16
        L.ts5r_fp32_to_fp16.argtypes = [C.c_float]
        L.ts5r_dequantize_row.argtypes = [C.c_uint32, C.c_void_p, _f32p, C.c_int64]
        L.ts5r_cpu_open.restype = C.c_void_p
        L.ts5r_cpu_open.argtypes = [C.c_char_p, C.c_int, C.c_int]
        L.ts5r_cpu_forward.argtypes = [C.c_void_p, _i32p, C.c_int, C.c_int, C.c_void_p, C.c_int]
        L.ts5r_cpu_close.argtypes = [C.c_void_p]
        L.ts5r_sample_table.argtypes = [_f32p, C.c_int, C.c_int, C.c_float, C.c_float, C.c_int, C.c_uint64,
                                        C.c_int, _i32p]
        L.ts5r_check.argtypes = [C.c_char_p, C.c_int, C.c_int, C.POINTER(C.c_double)]
        L.ts5r_generate.argtypes = [C.c_char_p, C.c_char_p, C.c_int, C.c_int, _i32p, C.c_int, C.c_float, C.c_float,
                                    C.c_int, C.c_uint64, C.c_int, C.c_int, _i32p, _i32p]
        _ref = L
    return _ref
