"""Python front end of the gfx950 backend (``libloom_hip.so``).

Mirrors the reference's kernel functions one for one -- same names, same
tensor arguments in the same order, same ``tile_*`` block-size parameters --
and calls the C ABI declared in ``include/loom_hip.h`` through ctypes on
torch's current HIP stream.  Like the reference's Python API
(``lib/pipeline/__init__.py:97-98,129-130``) a failure raises
``RuntimeError`` (here the subclass ``LoomHipError``, carrying the ABI's
return code) with the library's message.

Tensors are torch tensors on a ROCm device: bf16 arguments as
``torch.bfloat16``, fp32 arguments as ``torch.float32``, contiguous.  There
is no CPU fallback: if the shared library is missing, importing this module
raises.
"""
from __future__ import annotations

import ctypes
import functools
import json
import math
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
# LOOM_HIP_LIB selects another build of the same library (the host-side
# sanitizer build used by tests/test_sanitizers.py)
LIB_PATH = os.environ.get("LOOM_HIP_LIB") or os.path.join(os.path.dirname(_HERE), "libloom_hip.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(f"loom_hip: {LIB_PATH} is not built (run __graft_entry__.build())")

_lib = ctypes.CDLL(LIB_PATH)

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_f32 = ctypes.c_float
_ERR = (ctypes.c_char_p, _sz)

_SIGS = {
    "loom_hip_matmul": [_vp] * 3 + [_i64] * 6 + [_vp, *_ERR],
    "loom_hip_batch_matmul": [_vp] * 3 + [_i64] * 8 + [_vp, *_ERR],
    "loom_hip_split_k_matmul_gather": [_vp] * 4 + [_sz] + [_i64] * 6 + [_vp, *_ERR],
    "loom_hip_attention": [_vp] * 4 + [_i64] * 4 + [_f32, ctypes.c_int] + [_i64] * 3
    + [_vp, *_ERR],
    "loom_hip_flash_decode": [_vp] * 5 + [_sz] + [_i64] * 4 + [_f32] + [_i64] * 3
    + [_vp, *_ERR],
    "loom_hip_flash_decode_noalloc": [_vp] * 4 + [_i64] * 4 + [_f32] + [_i64] * 3 + [_vp, *_ERR],
    "loom_hip_helion_mamba2_chunk_scan_kernel": [_vp] * 8 + [_i64] * 13 + [_vp, *_ERR],
    "loom_hip_ssd_chunk_cumsum": [_vp] * 3 + [_i64] * 4 + [_vp, *_ERR],
    "loom_hip_ssd_bmm_chunk": [_vp] * 3 + [_i64] * 5 + [_vp, *_ERR],
    "loom_hip_ssd_chunk_state_passing": [_vp] * 5 + [_i64] * 7 + [_vp, *_ERR],
    "loom_hip_ssd_prologue": [_vp] * 8 + [_i64] * 7 + [_vp, *_ERR],
}
# f16 twins: same arguments, 16-bit tensors in IEEE binary16
for _name in ("loom_hip_matmul", "loom_hip_batch_matmul", "loom_hip_split_k_matmul_gather",
              "loom_hip_attention", "loom_hip_flash_decode",
              "loom_hip_helion_mamba2_chunk_scan_kernel", "loom_hip_ssd_bmm_chunk",
              "loom_hip_ssd_chunk_state_passing", "loom_hip_ssd_prologue"):
    _SIGS[_name + "_f16"] = _SIGS[_name]
for _name, _args in _SIGS.items():
    _fn = getattr(_lib, _name)
    _fn.argtypes = _args
    _fn.restype = ctypes.c_int
_lib.loom_hip_split_k_workspace_bytes.argtypes = [_i64] * 4
_lib.loom_hip_split_k_workspace_bytes.restype = _sz
_lib.loom_hip_flash_decode_workspace_bytes.argtypes = [_i64] * 5
_lib.loom_hip_flash_decode_workspace_bytes.restype = _sz
_lib.loom_hip_version.restype = ctypes.c_char_p
_lib.loom_hip_materialize_variants.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p),
                                               ctypes.c_int, ctypes.c_char_p, _sz, *_ERR]
_lib.loom_hip_materialize_variants.restype = ctypes.c_int
_lib.loom_hip_parse_variant.argtypes = [ctypes.c_char_p, ctypes.c_char_p, _sz,
                                        ctypes.POINTER(_i64), *_ERR]
_lib.loom_hip_parse_variant.restype = ctypes.c_int
_lib.loom_hip_dispatch.argtypes = [ctypes.c_char_p, ctypes.POINTER(_vp), ctypes.c_int,
                                   ctypes.POINTER(_i64), ctypes.c_int, _f32, ctypes.c_int,
                                   _vp, _sz, _vp, *_ERR]
_lib.loom_hip_dispatch.restype = ctypes.c_int
_lib.loom_hip_dispatch_f16.argtypes = _lib.loom_hip_dispatch.argtypes
_lib.loom_hip_dispatch_f16.restype = ctypes.c_int
_lib.loom_hip_check_variant.argtypes = [ctypes.c_char_p, ctypes.POINTER(_i64), ctypes.c_int, *_ERR]
_lib.loom_hip_check_variant.restype = ctypes.c_int
_lib.loom_hip_workspace_bytes.argtypes = [ctypes.c_char_p, ctypes.POINTER(_i64), ctypes.c_int,
                                          ctypes.POINTER(_sz), *_ERR]
_lib.loom_hip_workspace_bytes.restype = ctypes.c_int
for _fn in ("loom_hip_constraint_scope", "loom_hip_preferred_block_sizes", "loom_hip_hw_spec"):
    getattr(_lib, _fn).argtypes = [ctypes.c_char_p, ctypes.POINTER(_i64), ctypes.c_int,
                                   ctypes.c_char_p, _sz, *_ERR]
    getattr(_lib, _fn).restype = ctypes.c_int

# MLIR ranked memref descriptors {allocated, aligned, offset, sizes[R], strides[R]}
# (loom_memref<R>_t in include/loom_hip.h)
MEMREF = {}
for _r in range(1, 6):
    MEMREF[_r] = type(f"loom_memref{_r}_t", (ctypes.Structure,), {"_fields_": [
        ("allocated", _vp), ("aligned", _vp), ("offset", _i64), ("sizes", _i64 * _r),
        ("strides", _i64 * _r)]})
_MP = {r: ctypes.POINTER(MEMREF[r]) for r in MEMREF}
# descriptor ranks of each function's arguments, in IR order
_RANKS = {"matmul": (2, 2, 2), "batch_matmul": (3, 3, 3), "split_k_matmul_gather": (2, 2, 2),
          "attention": (3, 3, 3, 3), "flash_decode": (3, 3, 3, 3),
          "helion_mamba2_chunk_scan_kernel": (5, 4, 4, 4, 4, 1, 5, 4)}
_CIFACE_TAIL = {"matmul": [_i64] * 3, "batch_matmul": [_i64] * 4,
                "split_k_matmul_gather": [_vp, _sz] + [_i64] * 3,
                "attention": [_f32, ctypes.c_int] + [_i64] * 3,
                "flash_decode": [_vp, _sz, _f32] + [_i64] * 3,
                "helion_mamba2_chunk_scan_kernel": [_i64] * 6}
_CIFACE = []
for _f, _ranks in _RANKS.items():
    for _sfx in ("", "_f16"):
        _n = "loom_hip_ciface_" + _f + _sfx
        getattr(_lib, _n).argtypes = [_MP[r] for r in _ranks] + _CIFACE_TAIL[_f] + [_vp, *_ERR]
        getattr(_lib, _n).restype = ctypes.c_int
        _CIFACE.append(_n)
for _n in ("loom_hip_dispatch_memref", "loom_hip_dispatch_memref_f16"):
    getattr(_lib, _n).argtypes = [ctypes.c_char_p, ctypes.POINTER(_vp), ctypes.c_int, _f32,
                                  ctypes.c_int, _vp, _sz, _vp, *_ERR]
    getattr(_lib, _n).restype = ctypes.c_int
_lib.loom_hip_check_memref.argtypes = [ctypes.c_char_p, ctypes.POINTER(_vp), ctypes.c_int,
                                       ctypes.c_int, _f32, *_ERR]
_lib.loom_hip_check_memref.restype = ctypes.c_int

_lib.loom_hip_peak_hbm_read.argtypes = [_vp, _sz, _vp, _vp, *_ERR]
_lib.loom_hip_peak_hbm_read.restype = ctypes.c_int
_lib.loom_hip_peak_mfma_bf16.argtypes = [_i64, _vp, ctypes.POINTER(ctypes.c_double), _vp, *_ERR]
_lib.loom_hip_peak_mfma_bf16.restype = ctypes.c_int
_lib.loom_hip_synth.argtypes = [_vp, _i64, ctypes.c_uint64, ctypes.c_int, _f32, _f32, ctypes.c_int,
                                _vp, *_ERR]
_lib.loom_hip_synth.restype = ctypes.c_int
_lib.loom_hip_hw_spec.argtypes = [ctypes.c_int, ctypes.c_char_p, _sz, *_ERR]
_lib.loom_hip_hw_spec.restype = ctypes.c_int

EXPORTED = tuple(_SIGS) + tuple(_CIFACE) + ("loom_hip_peak_hbm_read", "loom_hip_peak_mfma_bf16", "loom_hip_synth") + ("loom_hip_dispatch_memref",
                                            "loom_hip_dispatch_memref_f16",
                                            "loom_hip_check_memref") + ("loom_hip_split_k_workspace_bytes",
                           "loom_hip_flash_decode_workspace_bytes", "loom_hip_version",
                           "loom_hip_materialize_variants", "loom_hip_parse_variant",
                           "loom_hip_dispatch", "loom_hip_dispatch_f16", "loom_hip_check_variant",
                           "loom_hip_workspace_bytes",
                           "loom_hip_constraint_scope", "loom_hip_preferred_block_sizes", "loom_hip_hw_spec")

#: block-size symbols in the slot order of loom_hip_parse_variant's tiles[]
TILE_SYMBOLS = ("tile_b", "tile_m", "tile_n", "tile_k", "tile_s", "tile_h", "tile_c")

__version__ = _lib.loom_hip_version().decode()


class LoomHipError(RuntimeError):
    """A loom_hip entry point returned nonzero (``code``: 1 invalid argument,
    2 not built for gfx950, 3 HIP runtime error)."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed (code {code}): {msg}")
        self.code = code


def _call(name: str, *args):
    buf = ctypes.create_string_buffer(512)
    rc = getattr(_lib, name)(*args, buf, len(buf))
    if rc != 0:
        raise LoomHipError(name, rc, buf.value.decode(errors="replace"))


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


_bf16, _f16, _fp32 = torch.bfloat16, torch.float16, torch.float32


def _elt(t):
    """16-bit element type of a kernel call, from one of its 16-bit tensors:
    (torch dtype, entry-point suffix).  bf16 and f16 (the reference's own
    element type) are built."""
    if isinstance(t, torch.Tensor) and t.dtype == _f16:
        return _f16, "_f16"
    return _bf16, ""


# Tensor arguments of every function, in IR order: (name, kind, shape from
# the extents).  kind "e" is the 16-bit element type of the call; "s" a side
# tensor -- fp32 in the bf16 variant, f16 (the reference's own type,
# examples/mamba_chunk_scan/IR/00_from_helion_frontend.mlir:4) in the f16
# variant.  Extents are in loom_hip_dispatch's order.
_SPECS = {
    "matmul": lambda M, N, K: (("x", "e", (M, K)), ("y", "e", (K, N)), ("out", "e", (M, N))),
    "batch_matmul": lambda B, M, N, K: (("arg0", "e", (B, M, K)), ("arg1", "e", (B, K, N)),
                                        ("arg2", "e", (B, M, N))),
    "split_k_matmul_gather": lambda M, N, K: (("a", "e", (M, K)), ("b", "e", (K, N)),
                                              ("out", "e", (M, N))),
    "attention": lambda BH, Sq, Skv, D: (("k", "e", (BH, D, Skv)), ("v", "e", (BH, Skv, D)),
                                         ("q", "e", (BH, Sq, D)), ("out", "e", (BH, Sq, D))),
    "flash_decode": lambda B, H, D, S: (("k", "e", (B, D, S)), ("v", "e", (B, S, D)),
                                        ("q", "e", (B, H, D)), ("out", "e", (B, H, D))),
    "helion_mamba2_chunk_scan_kernel": lambda b, nc, H, G, Q, P, N: (
        ("cb", "e", (b, nc, G, Q, Q)), ("x", "e", (b, H, nc * Q, P)),
        ("dt", "s", (b, H, nc, Q)), ("dA_cumsum", "s", (b, H, nc, Q)),
        ("C", "e", (b, G, nc * Q, N)), ("D", "s", (H,)), ("prev_states_T", "s", (b, nc, H, N, P)),
        ("out", "e", (b, H, nc * Q, P))),
}


def _check_form(t, name: str, dtype: torch.dtype, shape) -> None:
    """Type, dtype, exact shape and contiguity of one argument.  Nothing
    reaches the C ABI unchecked: it takes raw pointers and cannot see a short
    buffer or a wrong element type."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected {dtype}, got {t.dtype}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: expected shape {tuple(shape)}, got {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")


def _check_device(t, name: str, device=None) -> int:
    """One argument is on the call's ROCm device; its device pointer."""
    if t.device.type != "cuda":
        raise ValueError(f"{name}: must be on a ROCm device, got {t.device}")
    if device is not None and t.device != device:
        raise ValueError(f"{name}: on {t.device}, the call's tensors are on {device}")
    return t.data_ptr()


def _check_tensor(t, name: str, dtype: torch.dtype, shape, device=None) -> int:
    _check_form(t, name, dtype, shape)
    return _check_device(t, name, device)


def _check_call(func: str, tensors, dims, e: torch.dtype):
    """Validates every tensor argument of `func` against its extents (the form
    of all of them first, then their devices); returns the device pointers in
    IR order."""
    spec = _SPECS[func](*dims)
    if len(tensors) != len(spec):
        raise ValueError(f"{func}: takes {len(spec)} tensors ({', '.join(n for n, _, _ in spec)}), "
                         f"got {len(tensors)}")
    side = _fp32 if e == _bf16 else _f16
    for t, (name, kind, shape) in zip(tensors, spec):
        _check_form(t, name, e if kind == "e" else side, shape)
    dev0 = tensors[0].device
    return [_check_device(t, name, dev0) for t, (name, _, _) in zip(tensors, spec)]


def _shape2(t, name):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
    return tuple(t.shape)


def _dims_of(func: str, tensors):
    """Extents of a call (loom_hip_dispatch's order), read from its inputs;
    _check_call then holds every tensor to them."""
    sh = [_shape2(t, f"tensor {i}") for i, t in enumerate(tensors)]
    need = {"matmul": 2, "split_k_matmul_gather": 2, "batch_matmul": 2, "attention": 3,
            "flash_decode": 3, "helion_mamba2_chunk_scan_kernel": 5}[func]
    if len(sh) < need:
        raise ValueError(f"{func}: expected at least {need} tensors, got {len(sh)}")
    rank = lambda i, r: len(sh[i]) == r or (_ for _ in ()).throw(  # noqa: E731
        ValueError(f"{func}: tensor {i} must have {r} dims, got shape {sh[i]}"))
    if func in ("matmul", "split_k_matmul_gather"):
        rank(0, 2), rank(1, 2)
        return [sh[0][0], sh[1][1], sh[0][1]]
    if func == "batch_matmul":
        rank(0, 3), rank(1, 3)
        return [sh[0][0], sh[0][1], sh[1][2], sh[0][2]]
    if func == "attention":
        rank(0, 3), rank(2, 3)
        return [sh[0][0], sh[2][1], sh[0][2], sh[0][1]]
    if func == "flash_decode":
        rank(0, 3), rank(2, 3)
        return [sh[0][0], sh[2][1], sh[0][1], sh[0][2]]
    rank(0, 5), rank(1, 4), rank(4, 4)
    b, nc, G, Q, _ = sh[0]
    return [b, nc, sh[1][1], G, Q, sh[1][3], sh[4][3]]


@functools.lru_cache(maxsize=256)
def _preferred(func: str, dims: tuple) -> dict:
    return preferred_block_sizes(func, list(dims))


def _tiles(func: str, dims, **given):
    """Tile arguments of a call: the values given, and for each left as None
    the library's preferred binding for these extents (always within every
    symbol's natural_ub)."""
    if any(v is None for v in given.values()):
        pref = _preferred(func, tuple(int(d) for d in dims))
        given = {k: pref[k] if v is None else v for k, v in given.items()}
    return [int(given[k]) for k in given]


def _out_like(out, shape, e, dev):
    return torch.empty(shape, dtype=e, device=dev) if out is None else out


# ---------------------------------------------------------------------------
# kernels (examples/<k>/IR/00_from_helion_frontend.mlir)
# ---------------------------------------------------------------------------

def matmul(x, y, out=None, *, tile_m=None, tile_n=None, tile_k=None):
    """@matmul (examples/mm/IR/00_from_helion_frontend.mlir:2): out = x . y.
    Tiles left as None take the preferred binding for the extents."""
    e, sfx = _elt(x)
    M, N, K = _dims_of("matmul", (x, y))
    out = _out_like(out, (M, N), e, x.device)
    ptrs = _check_call("matmul", (x, y, out), (M, N, K), e)
    t = _tiles("matmul", (M, N, K), tile_m=tile_m, tile_n=tile_n, tile_k=tile_k)
    _call("loom_hip_matmul" + sfx, *ptrs, M, N, K, *t, _stream(x))
    return out


def batch_matmul(arg0, arg1, arg2=None, *, tile_b=None, tile_m=None, tile_n=None, tile_k=None):
    """@batch_matmul (examples/bmm_2Dmesh/IR/00_from_helion_frontend.mlir:4)."""
    e, sfx = _elt(arg0)
    dims = _dims_of("batch_matmul", (arg0, arg1))
    arg2 = _out_like(arg2, (dims[0], dims[1], dims[2]), e, arg0.device)
    ptrs = _check_call("batch_matmul", (arg0, arg1, arg2), dims, e)
    t = _tiles("batch_matmul", dims, tile_b=tile_b, tile_m=tile_m, tile_n=tile_n, tile_k=tile_k)
    _call("loom_hip_batch_matmul" + sfx, *ptrs, *dims, *t, _stream(arg0))
    return arg2


def split_k_workspace_bytes(M, N, K, tile_k) -> int:
    return int(_lib.loom_hip_split_k_workspace_bytes(M, N, K, tile_k))


def split_k_matmul_gather(a, b, out=None, partials=None, *, tile_m=None, tile_n=None,
                          tile_k=None):
    """@split_k_matmul_gather (examples/split_k_mm_gather/IR/00_from_helion_frontend.mlir:2).

    Returns (out [M,N] bf16, partials [S,M,N] fp32 -- the gathered K-slab
    products, S = ceil(K / tile_k))."""
    e, sfx = _elt(a)
    M, N, K = _dims_of("split_k_matmul_gather", (a, b))
    tile_m, tile_n, tile_k = _tiles("split_k_matmul_gather", (M, N, K), tile_m=tile_m,
                                    tile_n=tile_n, tile_k=tile_k)
    S = -(-K // tile_k) if tile_k > 0 else 1
    out = _out_like(out, (M, N), e, a.device)
    if partials is None:
        partials = torch.empty((max(S, 1), M, N), dtype=_fp32, device=a.device)
    _check_form(partials, "partials", _fp32, (max(S, 1), M, N))
    ptrs = _check_call("split_k_matmul_gather", (a, b, out), (M, N, K), e)
    pp = _check_device(partials, "partials", a.device)
    _call("loom_hip_split_k_matmul_gather" + sfx, *ptrs, pp, partials.numel() * 4, M, N, K,
          tile_m, tile_n, tile_k, _stream(a))
    return out, partials


def attention(k, v, q, out=None, *, scale=None, causal=False, tile_b=None, tile_m=None,
              tile_n=None):
    """@attention (examples/flashattn/IR/00_from_helion_frontend.mlir:4).

    k [BH,D,Skv] (keys transposed), v [BH,Skv,D], q [BH,Sq,D] -> out [BH,Sq,D].
    ``scale`` defaults to 1/sqrt(D)."""
    e, sfx = _elt(k)
    dims = _dims_of("attention", (k, v, q))
    BH, Sq, Skv, D = dims
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = _out_like(out, (BH, Sq, D), e, q.device)
    ptrs = _check_call("attention", (k, v, q, out), dims, e)
    t = _tiles("attention", dims, tile_b=tile_b, tile_m=tile_m, tile_n=tile_n)
    _call("loom_hip_attention" + sfx, *ptrs, BH, Sq, Skv, D, float(scale), int(bool(causal)), *t,
          _stream(q))
    return out


def flash_decode_workspace_bytes(B, H, D, S, tile_s) -> int:
    return int(_lib.loom_hip_flash_decode_workspace_bytes(B, H, D, S, tile_s))


def flash_decode_workspace(B, H, D, S, tile_s, device):
    """A flash_decode workspace (uint8 tensor) for these extents and tile_s."""
    return torch.empty(max(flash_decode_workspace_bytes(B, H, D, S, tile_s), 4),
                       dtype=torch.uint8, device=device)


def _check_workspace(ws, need, device, fn):
    if not isinstance(ws, torch.Tensor) or ws.device != device or ws.dtype != torch.uint8 or \
            not ws.is_contiguous() or ws.dim() != 1:
        raise ValueError(f"{fn}: workspace must be a contiguous 1-D uint8 tensor on {device}")
    if ws.numel() < need:
        raise ValueError(f"{fn}: workspace needs {need} bytes, got {ws.numel()}")
    return ws.data_ptr()


def flash_decode(k, v, q, out=None, workspace=None, *, scale=None, tile_b=None, tile_s=None,
                 tile_n=None, return_partials=False):
    """@flash_decode (examples/mqa_decode/IR/00_from_helion_frontend.mlir:6).

    k [B,D,S] (transposed), v [B,S,D], q [B,H,D] -> out [B,H,D].  With
    ``return_partials`` also returns the gathered (lse [ns,B,H], o [ns,B,H,D])."""
    e, sfx = _elt(k)
    dims = _dims_of("flash_decode", (k, v, q))
    B, H, D, S = dims
    tile_b, tile_s, tile_n = _tiles("flash_decode", dims, tile_b=tile_b, tile_s=tile_s,
                                    tile_n=tile_n)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = _out_like(out, (B, H, D), e, q.device)
    ptrs = _check_call("flash_decode", (k, v, q, out), dims, e)
    if workspace is None:
        workspace = flash_decode_workspace(B, H, D, S, tile_s, q.device)
    wp = _check_workspace(workspace, flash_decode_workspace_bytes(B, H, D, S, tile_s), q.device,
                          "flash_decode")
    _call("loom_hip_flash_decode" + sfx, *ptrs, wp, workspace.numel(), B, H, D, S, float(scale),
          tile_b, tile_s, tile_n, _stream(q))
    if not return_partials:
        return out
    ns = -(-S // tile_s)
    n_lse = ns * B * H
    off = (n_lse * 4 + 255) // 256 * 256
    lse = workspace[:n_lse * 4].view(torch.float32).view(ns, B, H)
    o = workspace[off:off + n_lse * D * 4].view(torch.float32).view(ns, B, H, D)
    return out, lse, o


#: bytes of the static device scratch loom_hip_flash_decode_noalloc keeps its
#: split partials in (one copy per device)
NOALLOC_SCRATCH_BYTES = 16 << 20


def flash_decode_noalloc(k, v, q, out, *, scale=None, tile_b=None, tile_s=None, tile_n=None):
    """flash_decode without a workspace: the split partials live in the
    library's static per-device scratch (``NOALLOC_SCRATCH_BYTES``), nothing is
    allocated (``out`` must be given).  Calls that overlap in time on one
    device share that scratch and race.  bf16 only."""
    dims = _dims_of("flash_decode", (k, v, q))
    B, H, D, S = dims
    tile_b, tile_s, tile_n = _tiles("flash_decode", dims, tile_b=tile_b, tile_s=tile_s,
                                    tile_n=tile_n)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    ptrs = _check_call("flash_decode", (k, v, q, out), dims, _bf16)
    _call("loom_hip_flash_decode_noalloc", *ptrs, B, H, D, S, float(scale), tile_b, tile_s, tile_n,
          _stream(q))
    return out


def helion_mamba2_chunk_scan_kernel(cb, x, dt, dA_cumsum, C, D, prev_states_T, out=None, *,
                                    tile_b=None, tile_h=None, tile_c=None, tile_m=None,
                                    tile_n=None, tile_k=None):
    """@helion_mamba2_chunk_scan_kernel
    (examples/mamba_chunk_scan/IR/00_from_helion_frontend.mlir:4).

    bf16 call: cb, x, C, out bf16; dt, dA_cumsum, D, prev_states_T fp32.
    f16 call (x in f16): every tensor f16, the reference's own signature."""
    e, sfx = _elt(x)
    f = "helion_mamba2_chunk_scan_kernel"
    dims = _dims_of(f, (cb, x, dt, dA_cumsum, C))
    b, nc, H, G, Q, P, N = dims
    out = _out_like(out, (b, H, nc * Q, P), e, x.device)
    ptrs = _check_call(f, (cb, x, dt, dA_cumsum, C, D, prev_states_T, out), dims, e)
    t = _tiles(f, dims, tile_b=tile_b, tile_h=tile_h, tile_c=tile_c, tile_m=tile_m, tile_n=tile_n,
               tile_k=tile_k)
    _call("loom_hip_" + f + sfx, *ptrs, *dims, *t, _stream(x))
    return out


# ---------------------------------------------------------------------------
# Mamba-2 SSD prologue (raw x, dt, A, B, C -> chunk_scan's inputs)
# ---------------------------------------------------------------------------

def ssd_prologue(x, dt, A, B, C, chunk_size, *, dA_cumsum=None, cb=None, prev_states_T=None):
    """x [b,H,L,P] bf16, dt [b,H,L] fp32 (post-softplus), A [H] fp32,
    B, C [b,G,L,N] bf16 -> (dt [b,H,c,Q] (a view of dt), dA_cumsum [b,H,c,Q],
    cb [b,c,G,Q,Q] bf16, prev_states_T [b,c,H,N,P] fp32).  With f16 x, B, C
    the cb output is f16; dA_cumsum and prev_states_T stay fp32."""
    e, sfx = _elt(x)
    if not isinstance(x, torch.Tensor) or x.dim() != 4 or not isinstance(B, torch.Tensor) \
            or B.dim() != 4:
        raise ValueError("ssd_prologue: x and B must be 4-D tensors")
    b, H, L, P = x.shape
    G, N = B.shape[1], B.shape[3]
    Q = int(chunk_size)
    if Q <= 0 or L % Q:
        raise ValueError("ssd_prologue: L must be a positive multiple of chunk_size")
    nc = L // Q
    dev = x.device
    if dA_cumsum is None:
        dA_cumsum = torch.empty((b, H, nc, Q), dtype=_fp32, device=dev)
    if cb is None:
        cb = torch.empty((b, nc, G, Q, Q), dtype=e, device=dev)
    if prev_states_T is None:
        prev_states_T = torch.empty((b, nc, H, N, P), dtype=_fp32, device=dev)
    spec = [(x, "x", e, (b, H, L, P)), (dt, "dt", _fp32, (b, H, L)), (A, "A", _fp32, (H,)),
            (B, "B", e, (b, G, L, N)), (C, "C", e, (b, G, L, N)),
            (dA_cumsum, "dA_cumsum", _fp32, (b, H, nc, Q)), (cb, "cb", e, (b, nc, G, Q, Q)),
            (prev_states_T, "prev_states_T", _fp32, (b, nc, H, N, P))]
    for a in spec:
        _check_form(*a)
    args = [_check_device(a[0], a[1], dev) for a in spec]
    _call("loom_hip_ssd_prologue" + sfx, *args, b, nc, H, G, Q, P, N, _stream(x))
    return dt.view(b, H, nc, Q), dA_cumsum, cb, prev_states_T

# ---------------------------------------------------------------------------
# materialization contract and by-name dispatch
# (lib/pipeline/src/loom_materialization_pipeline.cpp:81-192,251-270,
#  lib/passes/loom-opt/src/materialize.cpp:39-65,253-262)
# ---------------------------------------------------------------------------

FUNCTIONS = ("matmul", "batch_matmul", "split_k_matmul_gather", "attention", "flash_decode",
             "helion_mamba2_chunk_scan_kernel")


def materialize_variants(block_sizes_json: str, funcs=FUNCTIONS) -> list:
    """Variant names run_materialization emits for ``funcs`` under the
    solver's block-size JSON (``""`` = placeholder solver), in emission order.
    A rejected JSON raises ``RuntimeError`` with the reference's message."""
    names = [f.encode() for f in funcs]
    arr = (ctypes.c_char_p * max(len(names), 1))(*names)
    js = block_sizes_json.encode()
    cap = 4096 + 64 * len(js)
    while True:
        out = ctypes.create_string_buffer(cap)
        err = ctypes.create_string_buffer(512)
        rc = _lib.loom_hip_materialize_variants(js, arr, len(names), out, cap, err, len(err))
        if rc == 0:
            return [n for n in out.value.decode().split("\n") if n]
        msg = err.value.decode(errors="replace")
        if "output buffer needs" in msg:
            cap = int(msg.rsplit(" ", 2)[-2]) + 1
            continue
        raise LoomHipError("loom_hip_materialize_variants", rc, msg)


def parse_variant(name: str):
    """``"matmul__tile_k64__tile_m128__tile_n128"`` -> ``("matmul",
    {"tile_k": 64, "tile_m": 128, "tile_n": 128})``."""
    func = ctypes.create_string_buffer(len(name) + 1)
    tiles = (_i64 * len(TILE_SYMBOLS))()
    err = ctypes.create_string_buffer(512)
    rc = _lib.loom_hip_parse_variant(name.encode(), func, len(func), tiles, err, len(err))
    if rc != 0:
        raise LoomHipError("loom_hip_parse_variant", rc, err.value.decode(errors="replace"))
    return func.value.decode(), {s: int(t) for s, t in zip(TILE_SYMBOLS, tiles) if t >= 0}


def workspace_bytes(variant: str, dims) -> int:
    """Bytes of the workspace ``dispatch`` needs for a materialized variant at
    these extents (loom_hip_workspace_bytes): split-K's partials, decode's
    (lse_s, o_s), 0 for the other functions."""
    d = (_i64 * max(len(dims), 1))(*[int(x) for x in dims])
    out = _sz(0)
    _call("loom_hip_workspace_bytes", variant.encode(), d, len(dims), ctypes.byref(out))
    return int(out.value)


def dispatch(variant: str, *tensors, workspace=None, scale=None, causal=False):
    """Runs the kernel a materialized variant name selects on ``tensors``
    (the function's memref arguments in IR order, outputs included) through
    ``loom_hip_dispatch``.  Every tensor is checked against the function's
    signature (dtype, shape, device, contiguity) before anything launches.
    split_k_matmul_gather and flash_decode allocate their workspace when none
    is given; it is returned with the output."""
    func, tiles = parse_variant(variant)
    if func not in _SPECS:
        raise LoomHipError("loom_hip_dispatch", 2, f"no gfx950 kernel for function '{func}'")
    dims = _dims_of(func, tensors)
    e = _elt(tensors[1] if func == "helion_mamba2_chunk_scan_kernel" else tensors[0])[0]
    ptrs = _check_call(func, tensors, dims, e)
    dev = tensors[0].device
    need = 0
    if (func == "split_k_matmul_gather" and "tile_k" in tiles) or \
            (func == "flash_decode" and "tile_s" in tiles):
        need = workspace_bytes(variant, dims)
    if workspace is None and need:
        workspace = torch.empty(max(need, 4), dtype=torch.uint8, device=dev)
    ws_ptr, ws_bytes = None, 0
    if workspace is not None:
        ws_ptr = _check_workspace(workspace, need, dev, "dispatch")
        ws_bytes = workspace.numel()
    if scale is None:
        d = dims[3] if func == "attention" else dims[2] if func == "flash_decode" else 1
        scale = 1.0 / math.sqrt(d)
    tarr = (_vp * max(len(ptrs), 1))(*ptrs)
    darr = (_i64 * max(len(dims), 1))(*dims)
    err = ctypes.create_string_buffer(512)
    disp = _lib.loom_hip_dispatch_f16 if e == _f16 else _lib.loom_hip_dispatch
    rc = disp(variant.encode(), tarr, len(ptrs), darr, len(dims), float(scale),
              int(bool(causal)), ws_ptr, ws_bytes, _stream(tensors[0]), err, len(err))
    if rc != 0:
        raise LoomHipError("loom_hip_dispatch", rc, err.value.decode(errors="replace"))
    return tensors[-1], workspace


# ---------------------------------------------------------------------------
# gfx950 block-size constraints (the solver's input) and validation
# ---------------------------------------------------------------------------

def check_variant(variant: str, dims) -> None:
    """Raises ``LoomHipError`` if ``loom_hip_dispatch`` would reject the
    variant for these extents; launches nothing."""
    darr = (_i64 * max(len(dims), 1))(*dims)
    err = ctypes.create_string_buffer(512)
    rc = _lib.loom_hip_check_variant(variant.encode(), darr, len(dims), err, len(err))
    if rc != 0:
        raise LoomHipError("loom_hip_check_variant", rc, err.value.decode(errors="replace"))


def _json_call(name, func, dims):
    darr = (_i64 * max(len(dims), 1))(*dims)
    out = ctypes.create_string_buffer(1 << 16)
    err = ctypes.create_string_buffer(512)
    rc = getattr(_lib, name)(func.encode(), darr, len(dims), out, len(out), err, len(err))
    if rc != 0:
        raise LoomHipError(name, rc, err.value.decode(errors="replace"))
    return json.loads(out.value.decode())


def constraint_scope(func: str, dims) -> dict:
    """The gfx950 constraint scope of ``func`` for these extents, in the
    reference's staged-ETG JSON shape (see include/loom_hip.h)."""
    return _json_call("loom_hip_constraint_scope", func, dims)


def preferred_block_sizes(func: str, dims) -> dict:
    """The binding this library runs fastest for these extents."""
    return _json_call("loom_hip_preferred_block_sizes", func, dims)


# ---------------------------------------------------------------------------
# MLIR memref descriptors: the _mlir_ciface_ form of every function
# ---------------------------------------------------------------------------

def memref(t: torch.Tensor, offset: int = 0, base: torch.Tensor = None, strides=None):
    """A ranked memref descriptor (``MEMREF[t.dim()]``) for tensor ``t``.  With
    ``base`` given, the descriptor's allocated/aligned pointer is ``base``'s
    and ``offset`` is ``t``'s element offset from it (``t`` must lie inside
    ``base``); ``strides`` overrides the strides (in elements)."""
    r = t.dim()
    d = MEMREF[r]()
    if base is None:
        ptr, off = t.data_ptr(), offset
    else:
        ptr = base.data_ptr()
        off = (t.data_ptr() - ptr) // t.element_size()
    d.allocated = d.aligned = ptr
    d.offset = off
    for i in range(r):
        d.sizes[i] = t.shape[i]
        d.strides[i] = (strides if strides is not None else t.stride())[i]
    return d


def _desc_array(descs):
    keep = list(descs)
    arr = (_vp * max(len(keep), 1))(*[ctypes.cast(ctypes.pointer(d), _vp) for d in keep])
    return arr, keep


def ciface(func: str, *descs, f16=False, workspace=None, workspace_bytes=0, scale=1.0,
           causal=False, stream=None, **tiles):
    """Calls ``loom_hip_ciface_<func>`` (``_f16`` with ``f16``) on memref
    descriptors in IR order; tiles as keywords (``tile_m=...``)."""
    name = "loom_hip_ciface_" + func + ("_f16" if f16 else "")
    fn = getattr(_lib, name)
    ptrs = [ctypes.pointer(d) for d in descs]
    order = {"matmul": ("tile_m", "tile_n", "tile_k"),
             "batch_matmul": ("tile_b", "tile_m", "tile_n", "tile_k"),
             "split_k_matmul_gather": ("tile_m", "tile_n", "tile_k"),
             "attention": ("tile_b", "tile_m", "tile_n"),
             "flash_decode": ("tile_b", "tile_s", "tile_n"),
             "helion_mamba2_chunk_scan_kernel": ("tile_b", "tile_h", "tile_c", "tile_m", "tile_n",
                                                 "tile_k")}[func]
    t = [int(tiles[k]) for k in order]
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream if torch.cuda.is_available() else None
    ws = workspace.data_ptr() if isinstance(workspace, torch.Tensor) else workspace
    wsb = workspace.numel() if isinstance(workspace, torch.Tensor) else workspace_bytes
    if func == "split_k_matmul_gather":
        args = [*ptrs, ws, wsb, *t]
    elif func == "attention":
        args = [*ptrs, float(scale), int(bool(causal)), *t]
    elif func == "flash_decode":
        args = [*ptrs, ws, wsb, float(scale), *t]
    else:
        args = [*ptrs, *t]
    _call(name, *args, stream)


def dispatch_memref(variant: str, *descs, f16=False, workspace=None, scale=1.0, causal=False,
                    stream=None):
    """Runs a materialized variant on memref descriptors through
    ``loom_hip_dispatch_memref`` (``_f16`` with ``f16``)."""
    arr, _keep = _desc_array(descs)
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream if torch.cuda.is_available() else None
    ws = workspace.data_ptr() if workspace is not None else None
    wsb = workspace.numel() if workspace is not None else 0
    fn = _lib.loom_hip_dispatch_memref_f16 if f16 else _lib.loom_hip_dispatch_memref
    err = ctypes.create_string_buffer(512)
    rc = fn(variant.encode(), arr, len(descs), float(scale), int(bool(causal)), ws, wsb, stream,
            err, len(err))
    if rc != 0:
        raise LoomHipError("loom_hip_dispatch_memref", rc, err.value.decode(errors="replace"))


def check_memref(variant: str, *descs, f16=False, scale=1.0):
    """Raises ``LoomHipError`` if ``loom_hip_dispatch_memref`` would reject the
    call; launches nothing (no GPU needed)."""
    arr, _keep = _desc_array(descs)
    err = ctypes.create_string_buffer(512)
    rc = _lib.loom_hip_check_memref(variant.encode(), arr, len(descs), int(bool(f16)),
                                    float(scale), err, len(err))
    if rc != 0:
        raise LoomHipError("loom_hip_check_memref", rc, err.value.decode(errors="replace"))


# ---------------------------------------------------------------------------
# on-box ceilings
# ---------------------------------------------------------------------------

def peak_hbm_read(buf: torch.Tensor, sink: torch.Tensor) -> None:
    """Streams ``buf`` (a contiguous ROCm tensor) once through
    ``loom_hip_peak_hbm_read`` on the current stream."""
    _call("loom_hip_peak_hbm_read", buf.data_ptr(), buf.numel() * buf.element_size(),
          sink.data_ptr(), _stream(buf))


def peak_mfma_bf16(iters: int, sink: torch.Tensor) -> float:
    """Runs ``loom_hip_peak_mfma_bf16`` on the current stream; returns the FLOP
    it performs."""
    flop = ctypes.c_double()
    _call("loom_hip_peak_mfma_bf16", int(iters), sink.data_ptr(), ctypes.byref(flop),
          _stream(sink))
    return flop.value


def synth(shape, seed: int, dist: str = "normal", a: float = 0.0, b: float = 1.0,
          dtype: torch.dtype = torch.bfloat16, device="cuda") -> torch.Tensor:
    """A seeded synthetic tensor from ``loom_hip_synth``'s counter-based
    generator (bit-identical to the CPU oracle's ``oracle.synth``): dist
    "uniform" draws U[a, b), "normal" N(a, b) (mean a, standard deviation b);
    bf16 or float32."""
    if dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("synth: dtype must be torch.bfloat16 or torch.float32")
    d = {"uniform": 0, "normal": 1}.get(dist)
    if d is None:
        raise ValueError(f"synth: dist must be 'uniform' or 'normal', not {dist!r}")
    out = torch.empty(shape, dtype=dtype, device=device)
    _call("loom_hip_synth", out.data_ptr(), out.numel(), int(seed) & ((1 << 64) - 1), d,
          float(a), float(b), int(dtype == torch.bfloat16), _stream(out))
    return out


def hw_spec(device: int = -1) -> dict:
    """The MI355X machine model behind the constraint scopes
    (``loom_hip_hw_spec``); with ``device`` >= 0 also that device's
    reported properties."""
    buf = ctypes.create_string_buffer(1 << 14)
    _call("loom_hip_hw_spec", int(device), buf, len(buf))
    return json.loads(buf.value.decode())
