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
import math
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "libloom_hip.so")

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
for _fn in ("loom_hip_constraint_scope", "loom_hip_preferred_block_sizes"):
    getattr(_lib, _fn).argtypes = [ctypes.c_char_p, ctypes.POINTER(_i64), ctypes.c_int,
                                   ctypes.c_char_p, _sz, *_ERR]
    getattr(_lib, _fn).restype = ctypes.c_int

EXPORTED = tuple(_SIGS) + ("loom_hip_split_k_workspace_bytes",
                           "loom_hip_flash_decode_workspace_bytes", "loom_hip_version",
                           "loom_hip_materialize_variants", "loom_hip_parse_variant",
                           "loom_hip_dispatch", "loom_hip_dispatch_f16", "loom_hip_check_variant",
                           "loom_hip_constraint_scope", "loom_hip_preferred_block_sizes")

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


def _need(t: torch.Tensor, name: str, dtype: torch.dtype, ndim: int) -> int:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: must be on a ROCm device, got {t.device}")
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected {dtype}, got {t.dtype}")
    if t.dim() != ndim:
        raise ValueError(f"{name}: expected {ndim} dims, got shape {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    return t.data_ptr()


_bf16, _f16, _fp32 = torch.bfloat16, torch.float16, torch.float32


def _elt(t):
    """16-bit element type of a kernel call, from one of its 16-bit tensors:
    (torch dtype, entry-point suffix).  bf16 and f16 (the reference's own
    element type) are built."""
    if isinstance(t, torch.Tensor) and t.dtype == _f16:
        return _f16, "_f16"
    return _bf16, ""


# ---------------------------------------------------------------------------
# kernels (examples/<k>/IR/00_from_helion_frontend.mlir)
# ---------------------------------------------------------------------------

def matmul(x, y, out=None, *, tile_m=128, tile_n=128, tile_k=64):
    """@matmul (examples/mm/IR/00_from_helion_frontend.mlir:2): out = x . y."""
    _e, _sfx = _elt(x)
    M, K = x.shape
    N = y.shape[1]
    if y.shape[0] != K:
        raise ValueError(f"matmul: inner dims differ: {tuple(x.shape)} . {tuple(y.shape)}")
    if out is None:
        out = torch.empty((M, N), dtype=_e, device=x.device)
    if tuple(out.shape) != (M, N):
        raise ValueError("matmul: out shape mismatch")
    _call("loom_hip_matmul" + _sfx, _need(x, "x", _e, 2), _need(y, "y", _e, 2),
          _need(out, "out", _e, 2), M, N, K, tile_m, tile_n, tile_k, _stream(x))
    return out


def batch_matmul(arg0, arg1, arg2=None, *, tile_b=1, tile_m=256, tile_n=256, tile_k=64):
    """@batch_matmul (examples/bmm_2Dmesh/IR/00_from_helion_frontend.mlir:4)."""
    _e, _sfx = _elt(arg0)
    B, M, K = arg0.shape
    N = arg1.shape[2]
    if tuple(arg1.shape[:2]) != (B, K):
        raise ValueError("batch_matmul: arg1 shape mismatch")
    if arg2 is None:
        arg2 = torch.empty((B, M, N), dtype=_e, device=arg0.device)
    if tuple(arg2.shape) != (B, M, N):
        raise ValueError("batch_matmul: arg2 shape mismatch")
    _call("loom_hip_batch_matmul" + _sfx, _need(arg0, "arg0", _e, 3), _need(arg1, "arg1", _e, 3),
          _need(arg2, "arg2", _e, 3), B, M, N, K, tile_b, tile_m, tile_n, tile_k,
          _stream(arg0))
    return arg2


def split_k_workspace_bytes(M, N, K, tile_k) -> int:
    return int(_lib.loom_hip_split_k_workspace_bytes(M, N, K, tile_k))


def split_k_matmul_gather(a, b, out=None, partials=None, *, tile_m=64, tile_n=64, tile_k=1024):
    """@split_k_matmul_gather (examples/split_k_mm_gather/IR/00_from_helion_frontend.mlir:2).

    Returns (out [M,N] bf16, partials [S,M,N] fp32 -- the gathered K-slab
    products, S = ceil(K / tile_k))."""
    _e, _sfx = _elt(a)
    M, K = a.shape
    N = b.shape[1]
    if b.shape[0] != K:
        raise ValueError("split_k_matmul_gather: inner dims differ")
    S = -(-K // tile_k) if tile_k > 0 else 0
    if out is None:
        out = torch.empty((M, N), dtype=_e, device=a.device)
    if partials is None:
        partials = torch.empty((max(S, 1), M, N), dtype=_fp32, device=a.device)
    _call("loom_hip_split_k_matmul_gather" + _sfx, _need(a, "a", _e, 2), _need(b, "b", _e, 2),
          _need(out, "out", _e, 2), _need(partials, "partials", _fp32, 3),
          partials.numel() * 4, M, N, K, tile_m, tile_n, tile_k, _stream(a))
    return out, partials


def attention(k, v, q, out=None, *, scale=None, causal=False, tile_b=1, tile_m=256,
              tile_n=64):
    """@attention (examples/flashattn/IR/00_from_helion_frontend.mlir:4).

    k [BH,D,Skv] (keys transposed), v [BH,Skv,D], q [BH,Sq,D] -> out [BH,Sq,D].
    ``scale`` defaults to 1/sqrt(D)."""
    _e, _sfx = _elt(k)
    BH, D, Skv = k.shape
    Sq = q.shape[1]
    if tuple(v.shape) != (BH, Skv, D) or tuple(q.shape) != (BH, Sq, D):
        raise ValueError("attention: k/v/q shapes disagree")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty((BH, Sq, D), dtype=_e, device=q.device)
    _call("loom_hip_attention" + _sfx, _need(k, "k", _e, 3), _need(v, "v", _e, 3),
          _need(q, "q", _e, 3), _need(out, "out", _e, 3), BH, Sq, Skv, D,
          float(scale), int(bool(causal)), tile_b, tile_m, tile_n, _stream(q))
    return out


def flash_decode_workspace_bytes(B, H, D, S, tile_s) -> int:
    return int(_lib.loom_hip_flash_decode_workspace_bytes(B, H, D, S, tile_s))


def flash_decode_workspace(B, H, D, S, tile_s, device):
    """A flash_decode workspace (uint8 tensor) for these extents and tile_s."""
    return torch.empty(max(flash_decode_workspace_bytes(B, H, D, S, tile_s), 4),
                       dtype=torch.uint8, device=device)


def flash_decode(k, v, q, out=None, workspace=None, *, scale=None, tile_b=1, tile_s=1024,
                 tile_n=128, return_partials=False):
    """@flash_decode (examples/mqa_decode/IR/00_from_helion_frontend.mlir:6).

    k [B,D,S] (transposed), v [B,S,D], q [B,H,D] -> out [B,H,D].  With
    ``return_partials`` also returns the gathered (lse [ns,B,H], o [ns,B,H,D])."""
    _e, _sfx = _elt(k)
    B, D, S = k.shape
    H = q.shape[1]
    if tuple(v.shape) != (B, S, D) or tuple(q.shape) != (B, H, D):
        raise ValueError("flash_decode: k/v/q shapes disagree")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty((B, H, D), dtype=_e, device=q.device)
    if workspace is None:
        workspace = flash_decode_workspace(B, H, D, S, tile_s, q.device)
    if workspace.device != q.device or workspace.dtype != torch.uint8 or \
            not workspace.is_contiguous():
        raise ValueError("flash_decode: workspace must be a contiguous uint8 tensor")
    _call("loom_hip_flash_decode" + _sfx, _need(k, "k", _e, 3), _need(v, "v", _e, 3),
          _need(q, "q", _e, 3), _need(out, "out", _e, 3), workspace.data_ptr(),
          workspace.numel(), B, H, D, S, float(scale), tile_b, tile_s, tile_n, _stream(q))
    if not return_partials:
        return out
    ns = -(-S // tile_s)
    n_lse = ns * B * H
    off = (n_lse * 4 + 255) // 256 * 256
    lse = workspace[:n_lse * 4].view(torch.float32).view(ns, B, H)
    o = workspace[off:off + n_lse * D * 4].view(torch.float32).view(ns, B, H, D)
    return out, lse, o


def helion_mamba2_chunk_scan_kernel(cb, x, dt, dA_cumsum, C, D, prev_states_T, out=None, *,
                                    tile_b=1, tile_h=1, tile_c=1, tile_m=256, tile_n=64,
                                    tile_k=64):
    """@helion_mamba2_chunk_scan_kernel
    (examples/mamba_chunk_scan/IR/00_from_helion_frontend.mlir:4)."""
    _e, _sfx = _elt(x)
    b, nc, G, Q, _ = cb.shape
    _, H, L, P = x.shape
    N = C.shape[-1]
    if L != nc * Q or tuple(C.shape) != (b, G, L, N) or tuple(dt.shape) != (b, H, nc, Q) \
            or tuple(dA_cumsum.shape) != (b, H, nc, Q) or tuple(D.shape) != (H,) \
            or tuple(prev_states_T.shape) != (b, nc, H, N, P):
        raise ValueError("helion_mamba2_chunk_scan_kernel: argument shapes disagree")
    if out is None:
        out = torch.empty((b, H, L, P), dtype=_e, device=x.device)
    _call("loom_hip_helion_mamba2_chunk_scan_kernel" + _sfx, _need(cb, "cb", _e, 5),
          _need(x, "x", _e, 4), _need(dt, "dt", _fp32, 4),
          _need(dA_cumsum, "dA_cumsum", _fp32, 4), _need(C, "C", _e, 4),
          _need(D, "D", _fp32, 1), _need(prev_states_T, "prev_states_T", _fp32, 5),
          _need(out, "out", _e, 4), b, nc, H, G, Q, P, N, tile_b, tile_h, tile_c,
          tile_m, tile_n, tile_k, _stream(x))
    return out


# ---------------------------------------------------------------------------
# Mamba-2 SSD prologue (raw x, dt, A, B, C -> chunk_scan's inputs)
# ---------------------------------------------------------------------------

def ssd_prologue(x, dt, A, B, C, chunk_size, *, dA_cumsum=None, cb=None, prev_states_T=None):
    """x [b,H,L,P] bf16, dt [b,H,L] fp32 (post-softplus), A [H] fp32,
    B, C [b,G,L,N] bf16 -> (dt [b,H,c,Q] (a view of dt), dA_cumsum [b,H,c,Q],
    cb [b,c,G,Q,Q] bf16, prev_states_T [b,c,H,N,P] fp32)."""
    _e, _sfx = _elt(x)
    b, H, L, P = x.shape
    G, N = B.shape[1], B.shape[3]
    Q = int(chunk_size)
    if L % Q:
        raise ValueError("ssd_prologue: L must be a multiple of chunk_size")
    nc = L // Q
    if tuple(dt.shape) != (b, H, L) or tuple(A.shape) != (H,) or tuple(B.shape) != (b, G, L, N) \
            or tuple(C.shape) != (b, G, L, N):
        raise ValueError("ssd_prologue: argument shapes disagree")
    dev = x.device
    if dA_cumsum is None:
        dA_cumsum = torch.empty((b, H, nc, Q), dtype=_fp32, device=dev)
    if cb is None:
        cb = torch.empty((b, nc, G, Q, Q), dtype=_e, device=dev)
    if prev_states_T is None:
        prev_states_T = torch.empty((b, nc, H, N, P), dtype=_fp32, device=dev)
    _call("loom_hip_ssd_prologue" + _sfx, _need(x, "x", _e, 4), _need(dt, "dt", _fp32, 3),
          _need(A, "A", _fp32, 1), _need(B, "B", _e, 4), _need(C, "C", _e, 4),
          _need(dA_cumsum, "dA_cumsum", _fp32, 4), _need(cb, "cb", _e, 5),
          _need(prev_states_T, "prev_states_T", _fp32, 5), b, nc, H, G, Q, P, N, _stream(x))
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


def _dims_of(func: str, tensors):
    if func in ("matmul", "split_k_matmul_gather"):
        (M, K), N = tensors[0].shape, tensors[1].shape[1]
        return [M, N, K]
    if func == "batch_matmul":
        (B, M, K), N = tensors[0].shape, tensors[1].shape[2]
        return [B, M, N, K]
    if func == "attention":
        BH, D, Skv = tensors[0].shape
        return [BH, tensors[2].shape[1], Skv, D]
    if func == "flash_decode":
        B, D, S = tensors[0].shape
        return [B, tensors[2].shape[1], D, S]
    if func == "helion_mamba2_chunk_scan_kernel":
        b, nc, G, Q, _ = tensors[0].shape
        _, H, _, P = tensors[1].shape
        return [b, nc, H, G, Q, P, tensors[4].shape[-1]]
    raise LoomHipError("loom_hip_dispatch", 2, f"no gfx950 kernel for function '{func}'")


def dispatch(variant: str, *tensors, workspace=None, scale=None, causal=False):
    """Runs the kernel a materialized variant name selects on ``tensors``
    (the function's memref arguments in IR order, outputs included) through
    ``loom_hip_dispatch``.  split_k_matmul_gather and flash_decode allocate
    their workspace when none is given; it is returned with the output."""
    func, tiles = parse_variant(variant)
    dims = _dims_of(func, tensors)
    ptrs = []
    for i, t in enumerate(tensors):
        if not isinstance(t, torch.Tensor) or t.device.type != "cuda" or not t.is_contiguous():
            raise ValueError(f"dispatch: tensor {i} must be a contiguous ROCm tensor")
        ptrs.append(t.data_ptr())
    dev = tensors[0].device
    if workspace is None and func == "split_k_matmul_gather" and "tile_k" in tiles:
        M, N, K = dims
        workspace = torch.empty(max(split_k_workspace_bytes(M, N, K, tiles["tile_k"]), 4),
                                dtype=torch.uint8, device=dev)
    if workspace is None and func == "flash_decode" and "tile_s" in tiles:
        B, H, D, S = dims
        workspace = flash_decode_workspace(B, H, D, S, tiles["tile_s"], dev)
    if scale is None:
        d = dims[3] if func in ("attention",) else dims[2] if func == "flash_decode" else 1
        scale = 1.0 / math.sqrt(d)
    tarr = (_vp * max(len(ptrs), 1))(*ptrs)
    darr = (_i64 * max(len(dims), 1))(*dims)
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    err = ctypes.create_string_buffer(512)
    disp = _lib.loom_hip_dispatch_f16 if _elt(tensors[0])[0] == _f16 else _lib.loom_hip_dispatch
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
    import json
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
