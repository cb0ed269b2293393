"""The memref-descriptor boundary without a GPU (loom_hip_check_memref runs
every check of loom_hip_dispatch_memref and launches nothing).

A `_mlir_ciface_` caller passes each memref argument as a ranked descriptor
{allocated, aligned, offset, sizes, strides}.  These tests build descriptors
through ctypes and pin:
  - argument order: every argument gets its own distinct extents, so the
    correct order validates and swapping any two descriptors is refused with
    a message naming an argument;
  - the element offset: it moves the data pointer by offset * element size
    (an offset of one 16-bit element breaks the 16-byte alignment the kernels
    require, eight elements keep it; fp32 side tensors move by 4 bytes);
  - layouts: the row-major contiguous one is accepted, any other stride
    (innermost or outer, transposed or padded) refused, size-1 dimensions
    free;
  - null pointers, negative offsets and the descriptor count.
"""
import itertools

import pytest

import loom_hip

BASE = 1 << 24   # a 16-byte-aligned stand-in address, never dereferenced


def desc(shape, offset=0, strides=None, aligned=BASE):
    r = len(shape)
    d = loom_hip.MEMREF[r]()
    d.allocated = d.aligned = aligned
    d.offset = offset
    st = []
    e = 1
    for s in reversed(shape):
        st.append(e)
        e *= s
    st = list(reversed(st)) if strides is None else strides
    for i in range(r):
        d.sizes[i] = shape[i]
        d.strides[i] = st[i]
    return d


# function -> (variant name, argument shapes with distinct extents per axis, f16 flag)
M, N, K = 96, 160, 224
CALLS = {
    "matmul": ("matmul__tile_k32__tile_m64__tile_n64", [(M, K), (K, N), (M, N)]),
    "batch_matmul": ("batch_matmul__tile_b1__tile_k32__tile_m64__tile_n64",
                     [(3, M, K), (3, K, N), (3, M, N)]),
    "split_k_matmul_gather": ("split_k_matmul_gather__tile_k64__tile_m64__tile_n64",
                              [(M, K), (K, N), (M, N)]),
    "attention": ("attention__tile_b1__tile_m64__tile_n64",
                  [(5, 128, 136), (5, 136, 128), (5, 72, 128), (5, 72, 128)]),
    "flash_decode": ("flash_decode__tile_b1__tile_n64__tile_s128",
                     [(3, 64, 520), (3, 520, 64), (3, 24, 64), (3, 24, 64)]),
    "helion_mamba2_chunk_scan_kernel": (
        "helion_mamba2_chunk_scan_kernel__tile_b1__tile_c1__tile_h1__tile_k64__tile_m64__tile_n32",
        # b2 c3 H8 G2 Q64 P32 N48
        [(2, 3, 2, 64, 64), (2, 8, 192, 32), (2, 8, 3, 64), (2, 8, 3, 64), (2, 2, 192, 48), (8,),
         (2, 3, 8, 48, 32), (2, 8, 192, 32)]),
}


@pytest.mark.parametrize("func", sorted(CALLS))
@pytest.mark.parametrize("f16", [False, True])
def test_correct_order_validates(func, f16):
    variant, shapes = CALLS[func]
    loom_hip.check_memref(variant, *[desc(s) for s in shapes], f16=f16)


@pytest.mark.parametrize("func", sorted(CALLS))
def test_any_swap_is_refused(func):
    variant, shapes = CALLS[func]
    names = [n for n, _, _ in loom_hip._SPECS[func](*[1] * {"matmul": 3, "batch_matmul": 4,
                                                             "split_k_matmul_gather": 3,
                                                             "attention": 4, "flash_decode": 4}
                                                    .get(func, 7))]
    swaps = 0
    for i, j in itertools.combinations(range(len(shapes)), 2):
        if shapes[i] == shapes[j]:
            continue   # same shape, same rank: a swap is invisible to any checker
        s = list(shapes)
        s[i], s[j] = s[j], s[i]
        if len(s[i]) != len(shapes[i]) or len(s[j]) != len(shapes[j]):
            continue   # a rank mismatch is a C type error for the typed ciface entry points
        with pytest.raises(RuntimeError) as ei:
            loom_hip.check_memref(variant, *[desc(x) for x in s])
        assert ei.value.code == 1
        assert any(f" {n}: " in str(ei.value) for n in names), str(ei.value)
        swaps += 1
    assert swaps > 0


def test_offset_moves_the_data_pointer_by_elements():
    """attention refuses tensors that are not 16-byte aligned (the GEMMs run
    a misaligned operand on their element-store kernel instead)."""
    variant, shapes = CALLS["attention"]
    ok = [desc(s) for s in shapes]
    for i in range(4):
        d = list(ok)
        d[i] = desc(shapes[i], offset=8)          # 16 bytes of bf16: still aligned
        loom_hip.check_memref(variant, *d)
        d[i] = desc(shapes[i], offset=1)          # 2 bytes: misaligned for the kernels
        with pytest.raises(RuntimeError) as ei:
            loom_hip.check_memref(variant, *d)
        assert ei.value.code == 1 and "aligned" in str(ei.value)
        d[i] = desc(shapes[i], offset=-8)
        with pytest.raises(RuntimeError, match="negative offset"):
            loom_hip.check_memref(variant, *d)


def test_side_tensor_offsets_follow_their_element_size():
    """mamba's prev_states_T is fp32 in the bf16 form (4-byte elements: an
    offset of 4 keeps 16-byte alignment, 2 breaks it) and f16 in the f16 form
    (2-byte elements: 8 keeps it, 4 breaks it)."""
    variant, shapes = CALLS["helion_mamba2_chunk_scan_kernel"]
    for f16, good, bad in ((False, 4, 2), (True, 8, 4)):
        d = [desc(s) for s in shapes]
        d[6] = desc(shapes[6], offset=good)
        loom_hip.check_memref(variant, *d, f16=f16)
        d[6] = desc(shapes[6], offset=bad)
        with pytest.raises(RuntimeError, match="aligned"):
            loom_hip.check_memref(variant, *d, f16=f16)


def test_layouts():
    variant, shapes = CALLS["matmul"]
    x, y, out = shapes
    good = [desc(x), desc(y), desc(out)]
    cases = {
        "innermost stride 2": desc(x, strides=[2 * K, 2]),
        "transposed": desc(x, strides=[1, M]),
        "padded rows": desc(x, strides=[K + 8, 1]),
    }
    for what, bad in cases.items():
        with pytest.raises(RuntimeError) as ei:
            loom_hip.check_memref(variant, bad, good[1], good[2])
        msg = str(ei.value)
        assert ei.value.code == 1 and "x: strides" in msg and "row-major" in msg, (what, msg)
        if what == "innermost stride 2":
            assert "innermost stride must be 1" in msg
    # dimensions of size 1 are never stepped over: their strides are free
    v1 = "matmul__tile_k32__tile_m1__tile_n64"
    loom_hip.check_memref(v1, desc((1, K), strides=[12345, 1]), desc((K, N)), desc((1, N),
                                                                                 strides=[7, 1]))


def test_null_and_count():
    variant, shapes = CALLS["matmul"]
    d = [desc(s) for s in shapes]
    with pytest.raises(RuntimeError, match="takes 3 memref descriptors"):
        loom_hip.check_memref(variant, *d[:2])
    d[1] = desc(shapes[1], aligned=0)
    with pytest.raises(RuntimeError, match="y: null aligned pointer"):
        loom_hip.check_memref(variant, *d)


def test_tiles_and_unknown_functions_checked_as_dispatch():
    _, shapes = CALLS["matmul"]
    d = [desc(s) for s in shapes]
    with pytest.raises(RuntimeError) as ei:
        loom_hip.check_memref("matmul__tile_k32__tile_m128__tile_n128", *d)   # 128 > M = 96
    assert ei.value.code == 1 and "natural_ub" in str(ei.value)
    with pytest.raises(RuntimeError) as ei:
        loom_hip.check_memref("conv2d__tile_m64", *d)
    assert ei.value.code == 2
