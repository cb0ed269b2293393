"""Fuzzing the host-side input handling of the C ABI (CPU only, nothing
launches): the block-size JSON reader behind loom_hip_materialize_variants,
the variant-name parser, every entry point's validation (through
loom_hip_check_variant) and the memref-descriptor unpacking (through
loom_hip_check_memref).  Every input must either be accepted or be refused
with a code and a message -- never crash, hang or read out of bounds.
tests/test_sanitizers.py runs this file again against the AddressSanitizer
+ UndefinedBehaviorSanitizer build of the library, where any out-of-bounds
access, signed overflow or invalid conversion aborts the run.

Inputs: the committed corpus tests/golden/json_corpus/ (edge cases of the
JSON grammar and of the reference's block-size contract,
lib/pipeline/src/loom_materialization_pipeline.cpp:81-192), byte-level
mutations of it, random JSON documents, random variant names and extents
(including negative, zero and 2^62-sized ones), and random descriptors.
Hypothesis runs derandomized, so every run replays the same examples.
"""
import glob
import json
import os

import pytest
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

import loom_hip
from tests.conftest import GOLDEN

CORPUS = sorted(glob.glob(os.path.join(GOLDEN, "json_corpus", "*.json")))
FUNCS = list(loom_hip.FUNCTIONS)
FUZZ = settings(max_examples=300, derandomize=True, deadline=None,
                suppress_health_check=[HealthCheck.too_slow])


def materialize(text):
    """Names or a LoomHipError with code 1; anything else fails the test."""
    try:
        return loom_hip.materialize_variants(text, FUNCS)
    except RuntimeError as e:
        assert getattr(e, "code", None) == 1, str(e)
        return None


@pytest.mark.parametrize("path", CORPUS, ids=[os.path.basename(p)[:-5] for p in CORPUS])
def test_corpus(path):
    text = open(path, encoding="utf-8").read()
    names = materialize(text)
    base = os.path.basename(path)[:-5]
    expect_ok = {"empty_object", "placeholder_empty", "one_binding", "binding_list", "unsat_null",
                 "all_key", "candidate_order", "integral_real", "unicode_escapes",
                 "duplicate_keys", "whitespace", "many_bindings",
                 "long_symbol", "int_min", "nul_in_key"}
    if base in expect_ok:
        assert names is not None, base
    else:
        assert names is None, (base, names)
    if base == "integral_real":
        assert names == ["matmul__tile_k32__tile_m64__tile_n64"]
    if base == "unsat_null":
        assert names == ["attention__tile_b1__tile_m64__tile_n64"]
    if base == "many_bindings":   # identical bindings: __combo<i> renaming
        assert len(names) == 200 and len(set(names)) == 200


def test_corpus_errors_carry_the_reference_messages():
    def err(text):
        with pytest.raises(RuntimeError) as ei:
            loom_hip.materialize_variants(text, FUNCS)
        return str(ei.value)
    assert "must be an integer" in err('{"matmul": {"tile_m": 1e300}}')
    assert "must be an integer" in err('{"matmul": {"tile_m": 64.5}}')
    assert "nesting too deep" in err('{"matmul": ' + "[" * 100 + "]" * 100 + "}")
    # 60 levels parse (the reader's limit is 64); the binding is still not a
    # binding object, so the contract, not the reader, refuses it
    assert "nesting" not in err('{"x": ' + "[" * 60 + "]" * 60 + "}")


@FUZZ
@given(st.sampled_from(CORPUS), st.lists(st.tuples(st.integers(0, 2), st.integers(0, 1 << 16),
                                                   st.integers(0, 255)), max_size=8))
def test_mutated_corpus(path, edits):
    data = bytearray(open(path, "rb").read())
    for op, pos, byte in edits:
        pos = pos % (len(data) + 1)
        if op == 0:
            data.insert(pos, byte)
        elif op == 1 and data:
            del data[min(pos, len(data) - 1)]
        elif data:
            data[min(pos, len(data) - 1)] = byte
    text = data.decode("utf-8", errors="replace").replace("\x00", "")
    materialize(text)


json_values = st.recursive(
    st.none() | st.booleans() | st.integers(-(1 << 70), 1 << 70) |
    st.floats(allow_nan=False) | st.text(max_size=12),
    lambda kids: st.lists(kids, max_size=4) |
    st.dictionaries(st.sampled_from(FUNCS + ["ALL", "__loom_candidate_order__", "tile_m",
                                             "tile_k", "x"]) | st.text(max_size=6),
                    kids, max_size=4),
    max_leaves=24)


@FUZZ
@given(json_values)
def test_random_documents(doc):
    materialize(json.dumps(doc))


tokens = st.sampled_from(["tile_m", "tile_n", "tile_k", "tile_b", "tile_s", "tile_h", "tile_c",
                          "tile_x", "combo", "d0i0", "x8_y1y8", "", "__", "_"])


@FUZZ
@given(st.sampled_from(FUNCS + ["conv2d", ""]),
       st.lists(st.tuples(tokens, st.one_of(st.integers(0, 1 << 40),
                                            st.just(10 ** 15), st.just(-1))), max_size=7),
       st.lists(st.integers(-(1 << 62), 1 << 62) | st.integers(-4, 4096), max_size=9))
def test_random_variants_and_extents(func, toks, dims):
    name = func + "".join(f"__{t}{v if v >= 0 else ''}" for t, v in toks)
    try:
        loom_hip.parse_variant(name)
    except RuntimeError as e:
        assert e.code == 1, str(e)
    try:
        loom_hip.check_variant(name, dims)
    except RuntimeError as e:
        assert e.code in (1, 2), str(e)


RANKS = {"matmul": (2, 2, 2), "batch_matmul": (3, 3, 3), "split_k_matmul_gather": (2, 2, 2),
         "attention": (3, 3, 3, 3), "flash_decode": (3, 3, 3, 3),
         "helion_mamba2_chunk_scan_kernel": (5, 4, 4, 4, 4, 1, 5, 4)}
VARIANT = {"matmul": "matmul__tile_k32__tile_m64__tile_n64",
           "batch_matmul": "batch_matmul__tile_b1__tile_k32__tile_m64__tile_n64",
           "split_k_matmul_gather": "split_k_matmul_gather__tile_k64__tile_m64__tile_n64",
           "attention": "attention__tile_b1__tile_m64__tile_n64",
           "flash_decode": "flash_decode__tile_b1__tile_n64__tile_s128",
           "helion_mamba2_chunk_scan_kernel":
               "helion_mamba2_chunk_scan_kernel__tile_b1__tile_c1__tile_h1__tile_k64__tile_m64"
               "__tile_n32"}
extents = st.integers(-3, 300) | st.sampled_from([0, 1, 1 << 30, (1 << 31) - 1, 1 << 31,
                                                  1 << 40, 1 << 62, -(1 << 62)])


@FUZZ
@given(st.sampled_from(sorted(RANKS)), st.data())
def test_random_descriptors(func, data):
    descs = []
    for r in RANKS[func]:
        d = loom_hip.MEMREF[r]()
        d.allocated = d.aligned = data.draw(st.sampled_from([0, 1 << 24, (1 << 24) + 2]))
        d.offset = data.draw(st.integers(-2, 64) | st.sampled_from([1 << 56, 1 << 62]))
        for i in range(r):
            d.sizes[i] = data.draw(extents)
            d.strides[i] = data.draw(extents)
        descs.append(d)
    if data.draw(st.booleans()):
        descs = descs[:data.draw(st.integers(0, len(descs)))]
    try:
        loom_hip.check_memref(VARIANT[func], *descs, f16=data.draw(st.booleans()))
    except RuntimeError as e:
        assert e.code in (1, 2), str(e)
