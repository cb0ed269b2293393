"""The C-ABI boundary without a GPU.

- libloom_hip.so loads and exports every function include/loom_hip.h declares;
- every entry point rejects bad arguments with a nonzero code and a message
  before anything is launched (validation runs on the host), mirroring the
  reference's error-string contract (lib/pipeline/__init__.py:97-98,129-130);
- workspace-size helpers match the layouts the header documents.
"""
import ctypes
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
    rc, msg = _call(lh, "loom_hip_matmul", FAKE, FAKE, FAKE, 64, 64, 64, 96, 96, 64, None)
    assert rc == 2 and "not built" in msg
    rc, msg = _call(lh, "loom_hip_matmul", None, FAKE, FAKE, 64, 64, 64, 64, 64, 64, None)
    assert rc == 1 and "null" in msg
    rc, msg = _call(lh, "loom_hip_matmul", FAKE, FAKE, FAKE, 0, 64, 64, 64, 64, 64, None)
    assert rc == 1
    rc, msg = _call(lh, "loom_hip_batch_matmul", FAKE, FAKE, FAKE, 2, 64, 64, 64, 0, 64, 64, 64,
                    None)
    assert rc == 1 and "tile_b" in msg


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
    rc, msg = _call(lh, "loom_hip_attention", *base, 0.1, 1, 1, 96, 64, None)
    assert rc == 2 and "tile_m" in msg
    rc, msg = _call(lh, "loom_hip_attention", FAKE, FAKE, FAKE, FAKE, 4, 128, 64, 128, 0.1, 1,
                    1, 128, 64, None)
    assert rc == 1 and "causal" in msg
    rc, msg = _call(lh, "loom_hip_attention", FAKE, FAKE, FAKE, FAKE, 4, 128, 128, 80, 0.1, 0,
                    1, 128, 64, None)
    assert rc == 2 and "head_dim" in msg
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
    rc, msg = _call(lh, "loom_hip_flash_decode", FAKE, FAKE, FAKE, FAKE, FAKE, need,
                    B, 64, D, S, 0.1, 1, ts, 64, None)
    assert rc == 2 and "heads" in msg
    rc, msg = _call(lh, "loom_hip_flash_decode", FAKE, FAKE, FAKE, FAKE, FAKE, need,
                    B, H, D, S, 0.1, 1, S + 8, 64, None)
    assert rc == 1


def test_mamba_rejections(lh):
    dims = [1, 2, 4, 1, 64, 64, 128]
    rc, msg = _call(lh, "loom_hip_helion_mamba2_chunk_scan_kernel", *([FAKE] * 8), *dims,
                    1, 4, 1, 64, 64, 64, None)
    assert rc == 1 and "tile_b, tile_h and tile_c" in msg
    rc, msg = _call(lh, "loom_hip_helion_mamba2_chunk_scan_kernel", *([FAKE] * 8), *dims,
                    1, 1, 1, 48, 64, 64, None)
    assert rc == 2 and "tile_m" in msg
    rc, msg = _call(lh, "loom_hip_helion_mamba2_chunk_scan_kernel", *([FAKE] * 8),
                    1, 2, 6, 4, 64, 64, 128, 1, 1, 1, 64, 64, 64, None)
    assert rc == 1 and "ngroups" in msg


def test_ssd_rejections(lh):
    # x, dt, A, B, C, dA_cumsum, cb, prev_states_T | b, c, H, G, Q, P, N
    rc, msg = _call(lh, "loom_hip_ssd_prologue", *([FAKE] * 8), 1, 2, 6, 4, 64, 64, 128, None)
    assert rc == 1 and "ngroups" in msg
    rc, msg = _call(lh, "loom_hip_ssd_prologue", *([FAKE] * 8), 1, 2, 4, 1, 8, 64, 128, None)
    assert rc == 2 and "multiples of 16" in msg
    rc, msg = _call(lh, "loom_hip_ssd_prologue", *([FAKE] * 8), 1, 2, 4, 1, 512, 64, 128, None)
    assert rc == 2 and "chunk_size <= 256" in msg
    rc, msg = _call(lh, "loom_hip_ssd_prologue", *([FAKE] * 8), 1, 2, 4, 1, 256, 64, 48, None)
    assert rc == 2 and "multiple of 32" in msg
    rc, msg = _call(lh, "loom_hip_ssd_chunk_state_passing", None, *([FAKE] * 4),
                    1, 2, 4, 1, 64, 64, 128, None)
    assert rc == 1 and "null" in msg
    rc, msg = _call(lh, "loom_hip_ssd_chunk_cumsum", FAKE, FAKE, FAKE, 1, 2, 4, 1024, None)
    assert rc == 2 and "512" in msg
