"""ctypes binding of liboracle.so, the C restatement (oracle/csrc/oracle.c)."""

from __future__ import annotations

import ctypes
from ctypes import POINTER, Structure, c_float, c_int, c_int32, c_uint64, c_void_p
from pathlib import Path

import numpy as np

from .model import DecodeConfig

LIB = Path(__file__).resolve().parent / "lib" / "liboracle.so"
_lib = None


class _Cfg(Structure):
    _fields_ = [
        ("n_layers", c_int), ("dim", c_int), ("n_heads", c_int), ("n_kv", c_int), ("head_dim", c_int),
        ("ffn_dim", c_int), ("vocab", c_int), ("eps", c_float), ("theta", c_float), ("act", c_int),
        ("plus_one", c_int), ("embed_scale", c_int), ("untied_head", c_int), ("rope_factor", c_float),
        ("rope_low_freq_factor", c_float), ("rope_high_freq_factor", c_float), ("rope_original_max_positions", c_int),
    ]


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            from . import build

            build.build()
        L = ctypes.CDLL(str(LIB))
        L.oracle_fill_normal_f16.argtypes = [c_void_p, c_uint64, c_uint64, c_uint64, c_float]
        L.oracle_fill_normal_f32.argtypes = [c_void_p, c_uint64, c_uint64, c_uint64, c_float]
        L.oracle_matvec_f16.argtypes = [c_void_p, c_void_p, c_void_p, c_int, c_int]
        L.oracle_matvec_q8b32.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int]
        L.oracle_matvec_f32.argtypes = [c_void_p, c_void_p, c_void_p, c_int, c_int]
        L.oracle_model_create.argtypes = [POINTER(_Cfg), c_int, c_uint64, c_float, c_float]
        L.oracle_model_inv_freq.argtypes = [c_void_p, c_void_p]
        L.oracle_model_create.restype = c_void_p
        L.oracle_model_destroy.argtypes = [c_void_p]
        L.oracle_model_step.argtypes = [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p]
        L.oracle_model_step.restype = c_int
        L.oracle_num_threads.restype = c_int
        L.oracle_set_num_threads.argtypes = [c_int]
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags.c_contiguous
    return a.ctypes.data


def fill_normal(shape, dtype, seed: int, tensor_id: int, std: float) -> np.ndarray:
    out = np.empty(shape, dtype=dtype)
    fn = lib().oracle_fill_normal_f16 if dtype == np.float16 else lib().oracle_fill_normal_f32
    fn(_p(out), out.size, seed, tensor_id, std)
    return out


def matvec_f16(W: np.ndarray, x: np.ndarray) -> np.ndarray:
    M, K = W.shape
    y = np.empty(M, np.float64)
    lib().oracle_matvec_f16(_p(W), _p(np.ascontiguousarray(x, np.float32)), _p(y), M, K)
    return y


def matvec_q8b32(q: np.ndarray, s: np.ndarray, x: np.ndarray) -> np.ndarray:
    M, K = q.shape
    y = np.empty(M, np.float64)
    lib().oracle_matvec_q8b32(_p(q), _p(s), _p(np.ascontiguousarray(x, np.float32)), _p(y), M, K)
    return y


def matvec_f32(W: np.ndarray, x: np.ndarray) -> np.ndarray:
    M, K = W.shape
    y = np.empty(M, np.float64)
    lib().oracle_matvec_f32(_p(W), _p(np.ascontiguousarray(x, np.float32)), _p(y), M, K)
    return y


def num_threads() -> int:
    return lib().oracle_num_threads()


class NativeDecoder:
    """Full-size greedy decoder (the C restatement of oracle.model.OracleDecoder)."""

    def __init__(self, cfg: DecodeConfig, max_ctx: int, seed: int, std: float = 0.02, embed_std: float | None = None):
        rs = cfg.rope_scaling or (0.0, 0.0, 0.0, 0)
        c = _Cfg(cfg.n_layers, cfg.dim, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.ffn_dim, cfg.vocab, cfg.eps,
                 cfg.rope_theta, 1 if cfg.act == "silu" else 0, int(cfg.plus_one), int(cfg.gemma_embed_scale),
                 int(not cfg.tie_embeddings), float(rs[0]), float(rs[1]), float(rs[2]), int(rs[3]))
        self.cfg, self.max_ctx = cfg, max_ctx
        self._m = lib().oracle_model_create(ctypes.byref(c), max_ctx, seed, std, embed_std or std)
        if not self._m:
            raise MemoryError("oracle_model_create failed")
        self.tokens = np.zeros(max_ctx + 1, np.int32)

    def inv_freq(self) -> np.ndarray:
        out = np.empty(self.cfg.head_dim // 2, np.float32)
        lib().oracle_model_inv_freq(self._m, _p(out))
        return out

    def close(self) -> None:
        if self._m:
            lib().oracle_model_destroy(self._m)
            self._m = None

    def __del__(self):
        self.close()

    def step(self, pos: int, want_logits: bool = False, sample: bool = True):
        logits = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        margin = np.zeros(1, np.float32)
        rc = lib().oracle_model_step(self._m, _p(self.tokens), pos, int(sample), None if logits is None else _p(logits),
                                     _p(margin))
        if rc != 0:
            raise ValueError(f"oracle_model_step({pos}) -> {rc}")
        return int(self.tokens[pos + 1]), float(margin[0]), logits

    def generate(self, prompt: list[int], n_new: int, on_step=None) -> tuple[list[int], list[float]]:
        P = len(prompt)
        self.tokens[:P] = prompt
        margins = []
        for pos in range(P + n_new - 1):
            _, m, _ = self.step(pos, sample=pos >= P - 1)
            if pos >= P - 1:
                margins.append(m)
            if on_step:
                on_step(pos)
        return [int(t) for t in self.tokens[P : P + n_new]], margins
