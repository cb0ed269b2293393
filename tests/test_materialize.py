"""Materialization contract and by-name dispatch (CPU only: nothing here
launches a kernel).

Golden names come from the reference's own committed IR: the functions that
enter its Materialize pass (examples/<ex>/IR/05_after_enumerate_broadcast.mlir)
and the variant names it emitted (06_after_canonicalize.mlir), extracted by
tests/golden/make_variant_names.py.  mm, bmm_2Dmesh, flashattn and
mamba_chunk_scan were materialized by the placeholder solver
(lib/passes/loom-opt/src/materialize.cpp:56-65); mqa_decode and
split_k_mm_gather carry other bindings, reproduced here through "ALL".
Accept/reject rules and messages follow
lib/pipeline/src/loom_materialization_pipeline.cpp:81-192,251-270.
"""
import ctypes
import json
import os

import pytest

import loom_hip

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "variant_names.json")


@pytest.fixture(scope="module")
def names():
    with open(GOLDEN) as f:
        return json.load(f)


@pytest.mark.parametrize("ex", ["mm", "bmm_2Dmesh", "flashattn", "mamba_chunk_scan"])
def test_placeholder_solver_matches_reference_ir(names, ex):
    g = names[ex]
    assert loom_hip.materialize_variants("", g["funcs"]) == g["variants"]


@pytest.mark.parametrize("ex,binding", [
    ("mqa_decode", {"tile_b": 1, "tile_s": 512, "tile_n": 512}),
    ("split_k_mm_gather", {"tile_m": 64, "tile_n": 32, "tile_k": 512}),
])
def test_all_binding_matches_reference_ir(names, ex, binding):
    g = names[ex]
    js = json.dumps({"ALL": binding})
    assert loom_hip.materialize_variants(js, g["funcs"]) == g["variants"]
    # the same names from one explicit entry per function
    js = json.dumps({f: binding for f in g["funcs"]})
    assert loom_hip.materialize_variants(js, g["funcs"]) == g["variants"]


def test_parse_variant_inverts_every_reference_name(names):
    for ex, g in names.items():
        for f, v in zip(g["funcs"], g["variants"]):
            func, tiles = loom_hip.parse_variant(v)
            assert func == f.split("__")[0]
            suffix = v[len(f):]
            toks = [t for t in suffix.split("__") if t]
            assert {t.rstrip("0123456789"): int(t[len(t.rstrip("0123456789")):])
                    for t in toks} == tiles, v


def test_suffix_sorted_by_symbol_name():
    js = json.dumps({"f": {"tile_n": 1, "tile_m": 2, "tile_k": 3}})
    assert loom_hip.materialize_variants(js, ["f"]) == ["f__tile_k3__tile_m2__tile_n1"]
    # a binding of no symbols keeps the bare name
    assert loom_hip.materialize_variants('{"f": {}}', ["f"]) == ["f"]


def test_binding_list_and_combo_renaming():
    js = json.dumps({"f": [{"tile_m": 64}, {"tile_m": 64}, {"tile_m": 128}, {"tile_m": 64}]})
    # clash at binding i -> "__combo<i+1>", counting on past taken names
    assert loom_hip.materialize_variants(js, ["f"]) == [
        "f__tile_m64", "f__tile_m64__combo2", "f__tile_m128", "f__tile_m64__combo4"]
    js = json.dumps({"f": [{"a": 1}, {"a": 1}, {"a": 1}]})
    assert loom_hip.materialize_variants(js, ["f"]) == ["f__a1", "f__a1__combo2",
                                                       "f__a1__combo3"]


def test_null_is_unsat_and_missing_functions_are_skipped():
    js = json.dumps({"a": None, "b": {"tile_m": 8}})
    assert loom_hip.materialize_variants(js, ["a", "b", "c"]) == ["b__tile_m8"]


def test_candidate_order_sorts_functions_stably():
    js = json.dumps({"__loom_candidate_order__": ["c", "a"],
                     "a": {"tile_m": 1}, "b": {"tile_m": 2}, "c": {"tile_m": 3},
                     "d": {"tile_m": 4}})
    assert loom_hip.materialize_variants(js, ["a", "b", "c", "d"]) == [
        "c__tile_m3", "a__tile_m1", "b__tile_m2", "d__tile_m4"]


def test_all_yields_to_explicit_bindings_and_resets_order():
    js = json.dumps({"__loom_candidate_order__": ["b"], "ALL": {"tile_m": 1},
                     "b": {"tile_m": 2}})
    # ALL binds a and c, the order becomes [a, c]; b (explicit) is unranked
    assert loom_hip.materialize_variants(js, ["a", "b", "c"]) == [
        "a__tile_m1", "c__tile_m1", "b__tile_m2"]


def test_integral_reals_are_integers():
    assert loom_hip.materialize_variants('{"f": {"tile_m": 64.0, "tile_n": 1e2}}', ["f"]) == [
        "f__tile_m64__tile_n100"]


@pytest.mark.parametrize("js,msg", [
    ("[1, 2]", "block_sizes_json must be a JSON object at the top level"),
    ('"x"', "block_sizes_json must be a JSON object at the top level"),
    ('{"f": 3}', "Value for key 'f' must be a JSON object, array of objects, or null"),
    ('{"f": "64"}', "Value for key 'f' must be a JSON object, array of objects, or null"),
    ('{"f": []}', "Value for key 'f' must not be an empty array"),
    ('{"f": [{"tile_m": 1}, 2]}', "Value for key 'f' at index 1 must be a JSON object"),
    ('{"f": {"tile_m": 64.5}}', "Value for symbol 'tile_m' in 'f' must be an integer"),
    ('{"f": {"tile_m": "64"}}', "Value for symbol 'tile_m' in 'f' must be an integer"),
    ('{"f": {"tile_m": null}}', "Value for symbol 'tile_m' in 'f' must be an integer"),
    ('{"f": [{"tile_m": true}]}', "Value for symbol 'tile_m' in 'f' must be an integer"),
    ('{"__loom_candidate_order__": "f"}',
     "Value for '__loom_candidate_order__' must be an array"),
    ('{"__loom_candidate_order__": ["f", 1]}',
     "Entries in '__loom_candidate_order__' must be strings"),
])
def test_rejections_carry_reference_messages(js, msg):
    with pytest.raises(RuntimeError) as ei:
        loom_hip.materialize_variants(js, ["f"])
    assert msg in str(ei.value)
    assert ei.value.code == 1


@pytest.mark.parametrize("js", ["{", '{"f": {"tile_m": 1}', '{"f" 1}', "{} x", "nul",
                                '{"f": {"tile_m": 01x}}'])
def test_malformed_json(js):
    with pytest.raises(RuntimeError, match="Failed to parse block_sizes_json: "):
        loom_hip.materialize_variants(js, ["f"])


def test_parse_variant_rejects_bad_tokens():
    assert loom_hip.parse_variant("matmul") == ("matmul", {})
    assert loom_hip.parse_variant("matmul__combo3__tile_m8") == ("matmul", {"tile_m": 8})
    for bad in ("__tile_m64", "matmul__tile_m", "matmul__tile_q64"):
        with pytest.raises(RuntimeError):
            loom_hip.parse_variant(bad)


FAKE = 256  # never dereferenced: every case below is rejected before a launch


def _dispatch_raw(variant, ntensors, dims):
    lib = loom_hip._lib
    tarr = (ctypes.c_void_p * max(ntensors, 1))(*([FAKE] * ntensors))
    darr = (ctypes.c_int64 * max(len(dims), 1))(*dims)
    err = ctypes.create_string_buffer(256)
    rc = lib.loom_hip_dispatch(variant.encode(), tarr, ntensors, darr, len(dims), 1.0, 0,
                               None, 0, None, err, len(err))
    return rc, err.value.decode()


def test_dispatch_rejections():
    rc, msg = _dispatch_raw("conv2d__tile_m64", 3, [64, 64, 64])
    assert rc == 2 and "conv2d" in msg
    rc, msg = _dispatch_raw("matmul__tile_m128__tile_n128", 3, [256, 256, 256])
    assert rc == 1 and "lacks tile_k" in msg
    rc, msg = _dispatch_raw("matmul__tile_k64__tile_m128__tile_n128", 2, [256, 256, 256])
    assert rc == 1 and "takes 3 tensors and 3 extents" in msg
    # the entry point's own validation answers through dispatch
    rc, msg = _dispatch_raw("matmul__tile_k64__tile_m40__tile_n64", 3, [256, 256, 256])
    assert rc == 1 and "multiple of 16" in msg  # neither MFMA-aligned nor the extent
    # the placeholder mamba variant binds tile_h=4, tile_c=8, which the
    # gfx950 kernel does not take
    rc, msg = _dispatch_raw("helion_mamba2_chunk_scan_kernel__tile_b1__tile_c8__tile_h4"
                            "__tile_k64__tile_m64__tile_n32", 8, [2, 8, 32, 4, 192, 160, 128])
    assert rc == 1


def test_materialize_output_buffer_growth():
    funcs = [f"f{i}" for i in range(400)]
    js = json.dumps({"ALL": [{"tile_m": v, "tile_n": v} for v in (16, 32, 64)]})
    out = loom_hip.materialize_variants(js, funcs)
    assert len(out) == 1200 and out[0] == "f0__tile_m16__tile_n16"
