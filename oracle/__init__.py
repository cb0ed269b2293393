"""numpy front end of the fp32 CPU oracle (``oracle/oracle.c``).

TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package; the product path (``loom-dataflow_amd``) never does.

bf16 tensors are carried as ``numpy.uint16`` arrays holding the raw bf16
bits; ``to_bf16`` / ``from_bf16`` convert (round-to-nearest-even).  Every
function mirrors one reference function and cites it in ``oracle.c``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# LOOM_ORACLE_LIB selects another build (the sanitizer build of tests/test_sanitizers.py)
_LIB_PATH = os.environ.get("LOOM_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")
_lib = None

_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_ptr = ctypes.c_void_p


def build(force: bool = False) -> str:
    """Compile liboracle.so with the Makefile next to this file."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-B" if force else "-s", "-C", _HERE, "liboracle.so"],
                       check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        for name, args in {
            "loom_oracle_matmul": [_ptr] * 3 + [_i64] * 6,
            "loom_oracle_batch_matmul": [_ptr] * 3 + [_i64] * 8,
            "loom_oracle_split_k_matmul_gather": [_ptr] * 4 + [_i64] * 6,
            "loom_oracle_attention": [_ptr] * 4 + [_i64] * 4 + [_f32, ctypes.c_int] + [_i64] * 3,
            "loom_oracle_flash_decode": [_ptr] * 6 + [_i64] * 4 + [_f32] + [_i64] * 3,
            "loom_oracle_mamba_chunk_scan": [_ptr] * 8 + [_i64] * 10,
            "loom_oracle_mamba_prologue": [_ptr] * 9 + [_i64] * 7,
            "loom_oracle_widen16": [_ptr, _ptr, _i64],
            "loom_oracle_round16": [_ptr, _ptr, _i64],
            "loom_oracle_set_element_type": [ctypes.c_int],
            "loom_oracle_synth": [_ptr, _i64, ctypes.c_uint64, ctypes.c_int, _f32, _f32,
                                  ctypes.c_int],
            "loom_oracle_synth_sqrt": [_ptr, _ptr, _i64],
        }.items():
            fn = getattr(_lib, name)
            fn.argtypes = args
            fn.restype = None if name in ("loom_oracle_widen16", "loom_oracle_round16",
                                          "loom_oracle_set_element_type",
                                          "loom_oracle_synth_sqrt") else ctypes.c_int
        _lib.loom_oracle_num_threads.restype = ctypes.c_int
    return _lib


def num_threads() -> int:
    return int(lib().loom_oracle_num_threads())


# --------------------------------------------------------------------------
# bf16 <-> fp32 (numpy, round to nearest even)
# --------------------------------------------------------------------------

def to_bf16(a) -> np.ndarray:
    """fp32 values -> raw bf16 bits (uint16), round-to-nearest-even."""
    f = np.ascontiguousarray(a, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def from_bf16(h) -> np.ndarray:
    """raw bf16 bits (uint16) -> fp32."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def to_f16(a) -> np.ndarray:
    """fp32 values -> raw IEEE f16 bits (uint16), round-to-nearest-even."""
    return np.ascontiguousarray(a, dtype=np.float32).astype(np.float16).view(np.uint16)


def from_f16(h) -> np.ndarray:
    """raw IEEE f16 bits (uint16) -> fp32 (exact)."""
    return np.ascontiguousarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


class element_type:
    """Context manager selecting the 16-bit format the oracle's functions read
    and write: ``with oracle.element_type("f16"): ...`` (default "bf16")."""

    def __init__(self, name: str):
        if name not in ("bf16", "f16"):
            raise ValueError(f"element type {name!r}: bf16 or f16")
        self.f16 = name == "f16"

    def __enter__(self):
        self.prev = lib().loom_oracle_element_type()
        lib().loom_oracle_set_element_type(int(self.f16))
        return self

    def __exit__(self, *exc):
        lib().loom_oracle_set_element_type(self.prev)
        return False


def widen16(h) -> np.ndarray:
    """raw 16-bit elements -> fp32 through the oracle's C conversion (current
    element type)."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().loom_oracle_widen16(_p(h), _p(out), h.size)
    return out


def round16(a) -> np.ndarray:
    """fp32 -> raw 16-bit elements through the oracle's C conversion."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().loom_oracle_round16(_p(a), _p(out), a.size)
    return out


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def _u16(a):
    a = np.ascontiguousarray(a)
    assert a.dtype == np.uint16, a.dtype
    return a


def _f32c(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _check(rc, what):
    if rc != 0:
        raise ValueError(f"oracle {what}: rejected arguments (rc={rc})")


# --------------------------------------------------------------------------
# kernels
# --------------------------------------------------------------------------

def matmul(x, y, tile_m=64, tile_n=64, tile_k=64):
    x, y = _u16(x), _u16(y)
    M, K = x.shape
    K2, N = y.shape
    assert K == K2
    out = np.empty((M, N), np.uint16)
    _check(lib().loom_oracle_matmul(_p(x), _p(y), _p(out), M, N, K,
                                    min(tile_m, M), min(tile_n, N), min(tile_k, K)), "matmul")
    return out


def batch_matmul(a0, a1, tile_b=1, tile_m=64, tile_n=64, tile_k=64):
    a0, a1 = _u16(a0), _u16(a1)
    B, M, K = a0.shape
    B2, K2, N = a1.shape
    assert B == B2 and K == K2
    out = np.empty((B, M, N), np.uint16)
    _check(lib().loom_oracle_batch_matmul(_p(a0), _p(a1), _p(out), B, M, N, K,
                                          min(tile_b, B), min(tile_m, M), min(tile_n, N),
                                          min(tile_k, K)), "batch_matmul")
    return out


def split_k_matmul_gather(a, b, tile_m=64, tile_n=64, tile_k=1024):
    """Returns (out bf16 [M,N], partials fp32 [S,M,N])."""
    a, b = _u16(a), _u16(b)
    M, K = a.shape
    K2, N = b.shape
    assert K == K2
    S = -(-K // tile_k)
    out = np.empty((M, N), np.uint16)
    partials = np.empty((S, M, N), np.float32)
    _check(lib().loom_oracle_split_k_matmul_gather(_p(a), _p(b), _p(out), _p(partials),
                                                   M, N, K, tile_m, tile_n, tile_k),
           "split_k_matmul_gather")
    return out, partials


def attention(k, v, q, scale, causal=False, tile_b=1, tile_m=64, tile_n=64):
    """k [BH,D,Skv], v [BH,Skv,D], q [BH,Sq,D] (bf16 bits) -> out [BH,Sq,D]."""
    k, v, q = _u16(k), _u16(v), _u16(q)
    BH, D, Skv = k.shape
    _, Sq, _ = q.shape
    assert v.shape == (BH, Skv, D) and q.shape == (BH, Sq, D)
    out = np.empty((BH, Sq, D), np.uint16)
    _check(lib().loom_oracle_attention(_p(k), _p(v), _p(q), _p(out), BH, Sq, Skv, D,
                                       float(scale), int(bool(causal)), min(tile_b, BH),
                                       min(tile_m, Sq), min(tile_n, Skv)), "attention")
    return out


def flash_decode(k, v, q, scale, tile_b=1, tile_s=512, tile_n=64):
    """k [B,D,S], v [B,S,D], q [B,H,D] -> (out [B,H,D], lse [ns,B,H], o [ns,B,H,D])."""
    k, v, q = _u16(k), _u16(v), _u16(q)
    B, D, S = k.shape
    _, H, _ = q.shape
    assert v.shape == (B, S, D) and q.shape == (B, H, D)
    ns = -(-S // tile_s)
    out = np.empty((B, H, D), np.uint16)
    lse = np.empty((ns, B, H), np.float32)
    o = np.empty((ns, B, H, D), np.float32)
    _check(lib().loom_oracle_flash_decode(_p(k), _p(v), _p(q), _p(out), _p(lse), _p(o),
                                          B, H, D, S, float(scale), tile_b, tile_s, tile_n),
           "flash_decode")
    return out, lse, o


def mamba_chunk_scan(cb, x, dt, dA_cumsum, C, D, prev_states_T,
                     tile_m=64, tile_n=64, tile_k=64):
    cb, x, C = _u16(cb), _u16(x), _u16(C)
    dt, dA, Dh, prev = _f32c(dt), _f32c(dA_cumsum), _f32c(D), _f32c(prev_states_T)
    b, nc, G, Q, _ = cb.shape
    _, H, L, P = x.shape
    N = C.shape[-1]
    assert L == nc * Q and C.shape == (b, G, L, N)
    assert dt.shape == (b, H, nc, Q) and dA.shape == (b, H, nc, Q)
    assert prev.shape == (b, nc, H, N, P) and Dh.shape == (H,)
    out = np.empty((b, H, L, P), np.uint16)
    _check(lib().loom_oracle_mamba_chunk_scan(_p(cb), _p(x), _p(dt), _p(dA), _p(C), _p(Dh),
                                              _p(prev), _p(out), b, nc, H, G, Q, P, N,
                                              min(tile_m, Q), min(tile_n, P), tile_k),
           "mamba_chunk_scan")
    return out


def mamba_prologue(x, dt, A, B, C, chunk_size):
    """Raw Mamba-2 inputs -> chunk_scan inputs (dt [b,H,c,Q], dA_cumsum, cb, prev_states_T).

    x [b,H,L,P] bf16 bits, dt [b,H,L] fp32 (post-softplus), A [H] fp32,
    B and C [b,G,L,N] bf16 bits.
    """
    x, B, C = _u16(x), _u16(B), _u16(C)
    dt, A = _f32c(dt), _f32c(A)
    b, H, L, P = x.shape
    _, G, _, N = B.shape
    Q = chunk_size
    assert L % Q == 0
    nc = L // Q
    dt_out = np.empty((b, H, nc, Q), np.float32)
    dA = np.empty((b, H, nc, Q), np.float32)
    cb = np.empty((b, nc, G, Q, Q), np.uint16)
    prev = np.empty((b, nc, H, N, P), np.float32)
    _check(lib().loom_oracle_mamba_prologue(_p(x), _p(dt), _p(A), _p(B), _p(C), _p(dt_out),
                                            _p(dA), _p(cb), _p(prev), b, nc, H, G, Q, P, N),
           "mamba_prologue")
    return dt_out, dA, cb, prev


def synth(shape, seed, dist="normal", a=0.0, b=1.0, bf16=True):
    """The measurement protocol's synthetic tensor: element i of stream
    `seed` from the counter-based generator (oracle.c, loom_oracle_synth).
    dist "uniform": U[a, b); "normal": N(a, b) (mean a, standard deviation
    b).  Returns bf16 bits (uint16) or float32, in C order."""
    n = int(np.prod(shape, dtype=np.int64))
    out = np.empty(shape, np.uint16 if bf16 else np.float32)
    d = {"uniform": 0, "normal": 1}[dist]
    _check(lib().loom_oracle_synth(_p(out), n, int(seed) & ((1 << 64) - 1), d, a, b, int(bf16)),
           "synth")
    return out


def synth_sqrt(x) -> np.ndarray:
    """The generator's integer-arithmetic square root (test hook)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().loom_oracle_synth_sqrt(_p(x), _p(out), x.size)
    return out
