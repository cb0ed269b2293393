"""The C-ABI boundary without a GPU.

- libloom_hip.so loads and exports every function include/loom_hip.h declares;
- every entry point rejects bad arguments with a nonzero code and a message
  before anything is launched (validation runs on the host), mirroring the
  reference's error-string contract (lib/pipeline/__init__.py:97-98,129-130);
- workspace-size helpers match the layouts the header documents.
"""
import ctypes
import json
import os
import re

import pytest

from tests.conftest import ROOT

HEADER = os.path.join(ROOT, "include", "loom_hip.h")
LIB = os.path.join(ROOT, "loom-dataflow_amd", "libloom_hip.so")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(loom_hip_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lh():
    import loom_hip
    return loom_hip


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    names = declared()
    assert len(names) >= 9
    for n in names:
        assert hasattr(lib, n), f"{n} declared in loom_hip.h but not exported"


def test_python_binding_covers_abi(lh):
    assert set(lh.EXPORTED) == set(declared())
    assert lh.__version__.startswith("loom_hip ")


FAKE = ctypes.c_void_p(256)  # never dereferenced: validation fails first


def _call(lh, name, *args):
    buf = ctypes.create_string_buffer(256)
    rc = getattr(lh._lib, name)(*args, buf, len(buf))
    return rc, buf.value.decode()


def test_matmul_rejections(lh):
    # tiles are multiples of 16 (the MFMA edge) or the whole extent
    rc, msg = _call(lh, "loom_hip_matmul", FAKE, FAKE, FAKE, 256, 256, 256, 40, 64, 64, None)
    assert rc == 1 and "multiple of 16" in msg
    rc, msg = _call(lh, "loom_hip_matmul", None, FAKE, FAKE, 64, 64, 64, 64, 64, 64, None)
    assert rc == 1 and "null" in msg
    rc, msg = _call(lh, "loom_hip_matmul", FAKE, FAKE, FAKE, 0, 64, 64, 64, 64, 64, None)
    assert rc == 1
    rc, msg = _call(lh, "loom_hip_batch_matmul", FAKE, FAKE, FAKE, 2, 64, 64, 64, 0, 64, 64, 64,
                    None)
    assert rc == 1 and "tile_b" in msg


# Every loom.sym is bounded by the extent of the loop it tiles (natural_ub,
# lib/passes/lcs/src/staged_etg_builder.cpp:1420-1430; e.g. upper_bound = 2048
# for tile_m of a 2048-row matmul, examples/mm/IR/00_from_helion_frontend.mlir:8).
NATURAL_UB_CASES = [
    # (entry point, args before the stream, offending symbol)
    ("loom_hip_matmul", [FAKE] * 3 + [48, 1024, 1024, 256, 256, 64], "tile_m"),
    ("loom_hip_matmul", [FAKE] * 3 + [1024, 100, 1024, 128, 128, 64], "tile_n"),
    ("loom_hip_matmul", [FAKE] * 3 + [1024, 1024, 64, 64, 64, 4096], "tile_k"),
    ("loom_hip_batch_matmul", [FAKE] * 3 + [4, 256, 256, 256, 8, 64, 64, 64], "tile_b"),
    ("loom_hip_batch_matmul", [FAKE] * 3 + [4, 100, 256, 256, 1, 128, 128, 64], "tile_m"),
    ("loom_hip_batch_matmul", [FAKE] * 3 + [4, 256, 256, 32, 1, 64, 64, 64], "tile_k"),
    ("loom_hip_split_k_matmul_gather", [FAKE] * 4 + [1 << 30, 48, 512, 1024, 64, 64, 128],
     "tile_m"),
    ("loom_hip_split_k_matmul_gather", [FAKE] * 4 + [1 << 30, 512, 512, 1024, 64, 64, 2048],
     "tile_k"),
    ("loom_hip_attention", [FAKE] * 4 + [4, 128, 128, 128, 0.1, 0, 1, 256, 64], "tile_m"),
    ("loom_hip_attention", [FAKE] * 4 + [4, 128, 128, 128, 0.1, 0, 1, 128, 256], "tile_n"),
    ("loom_hip_attention", [FAKE] * 4 + [4, 128, 128, 128, 0.1, 0, 8, 128, 64], "tile_b"),
    ("loom_hip_flash_decode", [FAKE] * 5 + [1 << 30, 2, 32, 128, 1024, 0.1, 4, 256, 64], "tile_b"),
    ("loom_hip_flash_decode", [FAKE] * 5 + [1 << 30, 2, 32, 128, 1024, 0.1, 1, 2048, 64],
     "tile_s"),
    ("loom_hip_flash_decode", [FAKE] * 5 + [1 << 30, 2, 32, 128, 1024, 0.1, 1, 256, 4096],
     "tile_n"),
    ("loom_hip_helion_mamba2_chunk_scan_kernel",
     [FAKE] * 8 + [1, 2, 4, 1, 64, 64, 128, 1, 1, 1, 64, 64, 99999], "tile_k"),
    ("loom_hip_helion_mamba2_chunk_scan_kernel",
     [FAKE] * 8 + [1, 2, 4, 1, 64, 64, 128, 1, 1, 1, 128, 64, 64], "tile_m"),
    ("loom_hip_helion_mamba2_chunk_scan_kernel",
     [FAKE] * 8 + [1, 2, 4, 1, 64, 32, 128, 1, 1, 1, 64, 64, 64], "tile_n"),
]


@pytest.mark.parametrize("name,args,sym", NATURAL_UB_CASES,
                         ids=[f"{c[0][9:]}-{c[2]}" for c in NATURAL_UB_CASES])
def test_tile_above_natural_ub_rejected(lh, name, args, sym):
    for suffix in ("", "_f16"):
        rc, msg = _call(lh, name + suffix, *args, None)
        assert rc == 1 and sym in msg, (name + suffix, rc, msg)


def test_whole_extent_tile_accepted(lh):
    """A tiled symbol takes a multiple of 16 up to its extent, or the extent
    itself (it runs on the smallest built tile covering it); any other value
    is rejected."""
    lh.check_variant("matmul__tile_k24__tile_m48__tile_n40", [48, 40, 24])
    lh.check_variant("matmul__tile_k24__tile_m48__tile_n64", [48, 300, 24])
    lh.check_variant("attention__tile_b1__tile_m40__tile_n40", [2, 40, 40, 64])
    lh.check_variant("helion_mamba2_chunk_scan_kernel__tile_b1__tile_c1__tile_h1__tile_k48"
                     "__tile_m48__tile_n32", [1, 2, 4, 1, 48, 32, 64])
    with pytest.raises(RuntimeError) as ei:
        lh.check_variant("matmul__tile_k24__tile_m48__tile_n40", [48, 300, 24])
    assert ei.value.code == 1 and "multiple of 16" in str(ei.value)
    with pytest.raises(RuntimeError) as ei:
        lh.check_variant("matmul__tile_k24__tile_m64__tile_n64", [48, 40, 24])
    assert ei.value.code == 1


def test_reference_emitted_variants_accepted(lh):
    """Every in-bounds binding the reference's Materialize pass emitted
    (tests/golden/variant_names.json, from examples/*/IR/06_after_canonicalize.mlir)
    passes validation at the example's own extents: split-K's
    __tile_k512__tile_m64__tile_n32 on 512x4096 . 4096x512 and mqa_decode's
    __tile_b1__tile_n512__tile_s512 on B16 H32 D128 S8192.  The other
    examples' emitted names carry placeholder sizes beyond their extents
    (materialize.cpp:56-65) and are rejected as such."""
    with open(os.path.join(os.path.dirname(__file__), "golden", "variant_names.json")) as f:
        names = json.load(f)
    for ex, dims in (("split_k_mm_gather", [512, 512, 4096]), ("mqa_decode", [16, 32, 128, 8192])):
        assert len(names[ex]["variants"]) >= 8
        for n in names[ex]["variants"]:
            lh.check_variant(n, dims)
    with pytest.raises(RuntimeError) as ei:
        lh.check_variant(names["mm"]["variants"][0], [2048, 256, 256])
    assert ei.value.code == 1 and "natural_ub" in str(ei.value)


def test_mamba_tile_k_bound(lh):
    """tile_k is bounded by the example's loom.sym upper_bound (8192), not by
    the chunk: tile_k = 256 at chunk_size 192 is a binding the reference
    accepts."""
    base = "helion_mamba2_chunk_scan_kernel__tile_b1__tile_c1__tile_h1__tile_k{}__tile_m64__tile_n32"
    dims = [2, 8, 32, 4, 192, 160, 128]
    lh.check_variant(base.format(256), dims)
    lh.check_variant(base.format(8192), dims)
    with pytest.raises(RuntimeError) as ei:
        lh.check_variant(base.format(8193), dims)
    assert ei.value.code == 1 and "tile_k" in str(ei.value)


def test_split_k_rejections(lh):
    need = lh.split_k_workspace_bytes(64, 64, 1024, 128)
    assert need == 8 * 64 * 64 * 4
    rc, msg = _call(lh, "loom_hip_split_k_matmul_gather", FAKE, FAKE, FAKE, FAKE, need - 4,
                    64, 64, 1024, 64, 64, 128, None)
    assert rc == 1 and "workspace" in msg
    rc, msg = _call(lh, "loom_hip_split_k_matmul_gather", FAKE, FAKE, FAKE, FAKE, need,
                    64, 64, 1024, 64, 64, 2048, None)
    assert rc == 1 and "tile_k" in msg


def test_attention_rejections(lh):
    args = dict(BH=4, Sq=128, Skv=128, D=128)
    base = [FAKE] * 4 + [args["BH"], args["Sq"], args["Skv"], args["D"]]
    rc, msg = _call(lh, "loom_hip_attention", *base, 0.1, 1, 1, 40, 64, None)
    assert rc == 1 and "tile_m" in msg and "multiple of 16" in msg
    rc, msg = _call(lh, "loom_hip_attention", FAKE, FAKE, FAKE, FAKE, 4, 128, 64, 128, 0.1, 1,
                    1, 128, 64, None)
    assert rc == 1 and "causal" in msg
    # any multiple of 8 up to 256 is built (on the 64, 128 or 256 kernel); others are not
    for bad in (100, 264, 512):
        rc, msg = _call(lh, "loom_hip_attention", FAKE, FAKE, FAKE, FAKE, 4, 128, 128, bad, 0.1, 0,
                        1, 128, 64, None)
        assert rc == 2 and "head_dim" in msg, bad
    rc, msg = _call(lh, "loom_hip_attention", *base, 0.1, 0, 5, 128, 64, None)
    assert rc == 1  # tile_b > BH


def test_flash_decode_rejections(lh):
    B, H, D, S, ts = 2, 32, 128, 1024, 256
    need = lh.flash_decode_workspace_bytes(B, H, D, S, ts)
    ns = S // ts
    assert need == (ns * B * H * 4 + 255) // 256 * 256 + ns * B * H * D * 4
    rc, msg = _call(lh, "loom_hip_flash_decode", FAKE, FAKE, FAKE, FAKE, FAKE, need - 1,
                    B, H, D, S, 0.1, 1, ts, 64, None)
    assert rc == 1 and "workspace" in msg
    for bad in (100, 264):
        rc, msg = _call(lh, "loom_hip_flash_decode", FAKE, FAKE, FAKE, FAKE, FAKE, need,
                        B, H, bad, S, 0.1, 1, ts, 64, None)
        assert rc == 2 and "head_dim" in msg, bad
    rc, msg = _call(lh, "loom_hip_flash_decode", FAKE, FAKE, FAKE, FAKE, FAKE, need,
                    B, H, D, S, 0.1, 1, S + 8, 64, None)
    assert rc == 1
    # the running max is taken before scaling: only a finite positive scale is valid
    for bad in (0.0, -0.1, float("nan"), float("inf")):
        rc, msg = _call(lh, "loom_hip_flash_decode", FAKE, FAKE, FAKE, FAKE, FAKE, need,
                        B, H, D, S, bad, 1, ts, 64, None)
        assert rc == 1 and "scale" in msg, bad


def test_flash_decode_noalloc_rejections(lh):
    """The allocation-free decode keeps its partials in a 16 MiB static
    scratch: a call needing more is refused before anything touches a device
    (the scratch lookup itself would fail here, without a GPU, with code 3)."""
    B, H, D, S = 32, 32, 128, 8192
    assert lh.flash_decode_workspace_bytes(B, H, D, S, 1024) <= lh.NOALLOC_SCRATCH_BYTES
    assert lh.flash_decode_workspace_bytes(B, H, D, S, 256) > lh.NOALLOC_SCRATCH_BYTES
    rc, msg = _call(lh, "loom_hip_flash_decode_noalloc", FAKE, FAKE, FAKE, FAKE, B, H, D, S, 0.1,
                    1, 256, 64, None)
    assert rc == 1 and "scratch" in msg, (rc, msg)
    # the workspace form's own checks run first too
    rc, msg = _call(lh, "loom_hip_flash_decode_noalloc", FAKE, FAKE, FAKE, FAKE, B, H, 100, S, 0.1,
                    1, 1024, 64, None)
    assert rc == 2 and "head_dim" in msg, (rc, msg)
    rc, msg = _call(lh, "loom_hip_flash_decode_noalloc", FAKE, FAKE, FAKE, FAKE, B, H, D, S, -1.0,
                    1, 1024, 64, None)
    assert rc == 1 and "scale" in msg, (rc, msg)


def test_mamba_rejections(lh):
    dims = [1, 2, 4, 1, 64, 64, 128]
    rc, msg = _call(lh, "loom_hip_helion_mamba2_chunk_scan_kernel", *([FAKE] * 8), *dims,
                    1, 4, 1, 64, 64, 64, None)
    assert rc == 1 and "tile_b, tile_h and tile_c" in msg
    rc, msg = _call(lh, "loom_hip_helion_mamba2_chunk_scan_kernel", *([FAKE] * 8), *dims,
                    1, 1, 1, 40, 64, 64, None)
    assert rc == 1 and "tile_m" in msg and "multiple of 16" in msg
    rc, msg = _call(lh, "loom_hip_helion_mamba2_chunk_scan_kernel", *([FAKE] * 8),
                    1, 2, 6, 4, 64, 64, 128, 1, 1, 1, 64, 64, 64, None)
    assert rc == 1 and "ngroups" in msg


def test_ssd_rejections(lh):
    # x, dt, A, B, C, dA_cumsum, cb, prev_states_T | b, c, H, G, Q, P, N
    rc, msg = _call(lh, "loom_hip_ssd_prologue", *([FAKE] * 8), 1, 2, 6, 4, 64, 64, 128, None)
    assert rc == 1 and "ngroups" in msg
    rc, msg = _call(lh, "loom_hip_ssd_prologue", *([FAKE] * 8), 1, 2, 4, 1, 8, 64, 128, None)
    assert rc == 2 and "multiples of 16" in msg
    rc, msg = _call(lh, "loom_hip_ssd_prologue", *([FAKE] * 8), 1, 2, 4, 1, 640, 64, 128, None)
    assert rc == 2 and "chunk_size <= 512" in msg
    rc, msg = _call(lh, "loom_hip_ssd_prologue", *([FAKE] * 8), 1, 2, 4, 1, 256, 64, 288, None)
    assert rc == 2 and "dstate <= 256" in msg
    rc, msg = _call(lh, "loom_hip_ssd_prologue", *([FAKE] * 8), 1, 2, 4, 1, 256, 64, 48, None)
    assert rc == 2 and "multiple of 32" in msg
    rc, msg = _call(lh, "loom_hip_ssd_chunk_state_passing", None, *([FAKE] * 4),
                    1, 2, 4, 1, 64, 64, 128, None)
    assert rc == 1 and "null" in msg
    rc, msg = _call(lh, "loom_hip_ssd_chunk_cumsum", FAKE, FAKE, FAKE, 1, 2, 4, 1024, None)
    assert rc == 2 and "512" in msg
    # headdim above 256: refused before any of the three stages launches
    rc, msg = _call(lh, "loom_hip_ssd_prologue", *([FAKE] * 8), 1, 2, 4, 1, 256, 272, 128, None)
    assert rc == 2 and "headdim <= 256" in msg, (rc, msg)


def test_workspace_bytes_by_variant(lh):
    """loom_hip_workspace_bytes: the per-function workspace sizes, reached by
    a materialized name (the reference's own split-K and mqa variants
    included), 0 for functions without a workspace, and its rejections."""
    with open(os.path.join(os.path.dirname(__file__), "golden", "variant_names.json")) as f:
        emitted = json.load(f)
    sk = emitted["split_k_mm_gather"]["variants"][0]
    assert lh.workspace_bytes(sk, (512, 512, 4096)) == lh.split_k_workspace_bytes(512, 512, 4096, 512)
    mqa = emitted["mqa_decode"]["variants"][0]
    assert lh.workspace_bytes(mqa, (16, 32, 128, 8192)) == \
        lh.flash_decode_workspace_bytes(16, 32, 128, 8192, 512)
    assert lh.workspace_bytes("flash_decode__tile_b1__tile_n64__tile_s1000", (2, 40, 96, 3001)) == \
        lh.flash_decode_workspace_bytes(2, 40, 96, 3001, 1000)
    assert lh.workspace_bytes("matmul__tile_k64__tile_m64__tile_n64", (64, 64, 64)) == 0
    assert lh.workspace_bytes("attention__tile_b1__tile_m64__tile_n64", (2, 64, 64, 128)) == 0
    assert lh.workspace_bytes("helion_mamba2_chunk_scan_kernel__tile_b1__tile_c1__tile_h1__tile_k64"
                              "__tile_m64__tile_n64", (1, 2, 4, 1, 64, 64, 128)) == 0
    for name, dims, code in (("conv2d__tile_m64", (1, 2, 3), 2),                       # no kernel
                             ("split_k_matmul_gather__tile_m64__tile_n64", (8, 8, 8), 1),  # tile_k
                             ("flash_decode__tile_s64", (1, 2, 64), 1),                # 3 extents
                             ("flash_decode__tile_s64", (1, 2, 64, 0), 1)):             # not positive
        with pytest.raises(lh.LoomHipError) as ei:
            lh.workspace_bytes(name, dims)
        assert ei.value.code == code, name
