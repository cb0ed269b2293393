"""gfx950 block-size constraint scopes (CPU only: nothing launches).

The scopes are written in the reference's constraint grammar
(lib/passes/lcs/inc/expr.h, constraint_expr.h).  `evaluate` below is an
interpreter of that published grammar; the tests check, over a grid of
candidate bindings per function and shape, that the scope's hard constraints
accept exactly the bindings the library itself accepts
(loom_hip_check_variant runs the entry point's own validation and launches
nothing), that the symbol set is the function's loom.sym set, and that the
preferred binding is legal.
"""
import itertools
import json

import pytest

import loom_hip


def evaluate(node, env):
    """Interpreter of the reference's Expr / ConstraintExpr JSON."""
    if node == "True":
        return True
    if node == "False":
        return False
    (op, arg), = node.items()
    if op == "Const":
        return arg
    if op == "Sym":
        return env[arg]
    if op in ("Add", "Sub", "Mul", "Div", "Min", "Max"):
        a, b = (evaluate(x, env) for x in arg)
        return {"Add": a + b, "Sub": a - b, "Mul": a * b, "Div": a // b,
                "Min": min(a, b), "Max": max(a, b)}[op]
    if op == "IfElse":
        return evaluate(arg["then_expr"] if evaluate(arg["cond"], env) else arg["else_expr"], env)
    if op == "And":
        return all(evaluate(x, env) for x in arg)
    if op == "Or":
        return any(evaluate(x, env) for x in arg)
    if op == "Not":
        return not evaluate(arg, env)
    if op in ("Eq", "Le", "Lt", "Ge", "Gt"):
        a, b = (evaluate(x, env) for x in arg)
        return {"Eq": a == b, "Le": a <= b, "Lt": a < b, "Ge": a >= b, "Gt": a > b}[op]
    if op == "InRange":
        x = evaluate(arg["x"], env)
        return evaluate(arg["lo"], env) <= x <= evaluate(arg["hi"], env)
    if op == "Divisible":
        return evaluate(arg["x"], env) % evaluate(arg["by"], env) == 0
    raise AssertionError(f"unknown node {op}")


# function -> (loom.sym symbols in the example IR, extents cases)
CASES = {
    "matmul": (["tile_m", "tile_n", "tile_k"], [(1024, 1024, 1024), (2048, 256, 256), (48, 40, 24)]),
    "batch_matmul": (["tile_b", "tile_m", "tile_n", "tile_k"], [(16, 2048, 2048, 2048), (2, 96, 80, 64)]),
    "split_k_matmul_gather": (["tile_m", "tile_n", "tile_k"], [(512, 512, 16384), (48, 96, 1000)]),
    "attention": (["tile_b", "tile_m", "tile_n"], [(128, 4096, 4096, 128), (3, 1000, 1000, 64),
                                                   (2, 300, 300, 96), (2, 500, 500, 256)]),
    "flash_decode": (["tile_b", "tile_s", "tile_n"], [(32, 32, 128, 8192), (3, 5, 64, 1000),
                                                       (2, 64, 128, 2048), (2, 8, 40, 1000),
                                                       (2, 8, 256, 1000)]),
    "helion_mamba2_chunk_scan_kernel": (["tile_m", "tile_n", "tile_k", "tile_c", "tile_b", "tile_h"],
                                        [(4, 16, 32, 1, 256, 64, 128), (2, 8, 32, 4, 192, 160, 128),
                                         (1, 2, 4, 1, 512, 64, 256), (1, 2, 3, 1, 264, 40, 136)]),
}
GRID = [1, 16, 48, 64, 96, 128, 192, 256, 1024]
SMALL = [1, 2]


def _variant(func, binding):
    return func + "".join(f"__{k}{v}" for k, v in sorted(binding.items()))


@pytest.mark.parametrize("func", sorted(CASES))
def test_scope_accepts_exactly_what_the_kernels_build(func):
    syms, shapes = CASES[func]
    for dims in shapes:
        scope = loom_hip.constraint_scope(func, dims)
        assert scope["variant_name"] == func
        meta = scope["constraint_scope"]["metadata"]
        assert sorted(meta["symbols"]) == sorted(syms)
        hard = scope["constraint_scope"]["hard_constraints"]
        # every symbol takes grid values plus its natural upper bound (+1)
        values = {s: sorted(set((SMALL if s in ("tile_b", "tile_h", "tile_c") else GRID) +
                                [meta["symbols"][s]["natural_ub"],
                                 meta["symbols"][s]["natural_ub"] + 1]))
                  for s in syms}
        accepted = 0
        for combo in itertools.product(*(values[s] for s in syms)):
            env = dict(zip(syms, combo))
            legal = all(evaluate(c, env) for c in hard)
            try:
                loom_hip.check_variant(_variant(func, env), dims)
                built = True
            except RuntimeError as e:
                assert e.code in (1, 2), str(e)
                built = False
            assert legal == built, (func, dims, env, legal, built)
            accepted += legal
        assert accepted > 0, (func, dims)


@pytest.mark.parametrize("func", sorted(CASES))
def test_preferred_binding_is_legal(func):
    syms, shapes = CASES[func]
    for dims in shapes:
        pref = loom_hip.preferred_block_sizes(func, dims)
        assert sorted(pref) == sorted(syms)
        hard = loom_hip.constraint_scope(func, dims)["constraint_scope"]["hard_constraints"]
        assert all(evaluate(c, pref) for c in hard), (func, dims, pref)
        loom_hip.check_variant(_variant(func, pref), dims)


def test_preferred_bindings_at_baseline_shapes():
    """The tunings the bench runs."""
    assert loom_hip.preferred_block_sizes("batch_matmul", (16, 2048, 2048, 2048)) == {
        "tile_b": 1, "tile_k": 64, "tile_m": 256, "tile_n": 256}
    assert loom_hip.preferred_block_sizes("attention", (128, 4096, 4096, 128))["tile_m"] == 256
    assert loom_hip.preferred_block_sizes("flash_decode", (32, 32, 128, 8192))["tile_s"] == 1024
    # split-K: enough K slabs for a workgroup per CU (BASELINE itself fixes 16 slabs)
    sk = loom_hip.preferred_block_sizes("split_k_matmul_gather", (512, 512, 16384))
    assert (sk["tile_m"], sk["tile_n"], sk["tile_k"]) == (128, 128, 1024)
    assert loom_hip.preferred_block_sizes("matmul", (1024, 1024, 1024))["tile_m"] == 64
    m = loom_hip.preferred_block_sizes("helion_mamba2_chunk_scan_kernel", (4, 16, 32, 1, 256, 64, 128))
    assert (m["tile_m"], m["tile_n"]) == (256, 64)


def test_scope_json_round_trips_into_block_sizes_json():
    """A preferred binding is a valid block_sizes_json entry for the
    materialization contract, and its variant name parses back."""
    dims = (16, 2048, 2048, 2048)
    pref = loom_hip.preferred_block_sizes("batch_matmul", dims)
    names = loom_hip.materialize_variants(json.dumps({"batch_matmul": pref}), ["batch_matmul"])
    assert names == ["batch_matmul__tile_b1__tile_k64__tile_m256__tile_n256"]
    assert loom_hip.parse_variant(names[0]) == ("batch_matmul", pref)
    loom_hip.check_variant(names[0], dims)


def test_unsupported_shapes_and_functions():
    for d in (100, 264):   # head_dim: a multiple of 8 up to 256
        with pytest.raises(RuntimeError) as ei:
            loom_hip.constraint_scope("attention", (4, 128, 128, d))
        assert ei.value.code == 2
        with pytest.raises(RuntimeError) as ei:
            loom_hip.constraint_scope("flash_decode", (4, 8, d, 1024))
        assert ei.value.code == 2
    loom_hip.constraint_scope("flash_decode", (4, 8, 136, 1001))   # any S at any built D
    # chunk scan: chunk_size up to 512, dstate up to 256 (multiples of 8)
    for dims in ((1, 2, 4, 1, 520, 64, 128), (1, 2, 4, 1, 256, 64, 264),
                 (1, 2, 4, 1, 260, 64, 128)):
        with pytest.raises(RuntimeError) as ei:
            loom_hip.constraint_scope("helion_mamba2_chunk_scan_kernel", dims)
        assert ei.value.code == 2, dims
    assert loom_hip.preferred_block_sizes("attention", (8, 4096, 4096, 256))["tile_m"] == 128
    with pytest.raises(RuntimeError) as ei:
        loom_hip.constraint_scope("conv2d", (1, 2, 3))
    assert ei.value.code == 2
    with pytest.raises(RuntimeError) as ei:
        loom_hip.constraint_scope("matmul", (1, 2))
    assert ei.value.code == 1
    # the TT 32-alignment becomes the 16-element MFMA edge, and every symbol is
    # bounded by its extent (natural_ub): on a 48x40 GEMM the whole extents
    # are legal (they run as one 64x64 tile), 64 exceeds them, 32 and 16 are
    # multiples of 16, 24 is neither that nor an extent
    hard = loom_hip.constraint_scope("matmul", (48, 40, 24))["constraint_scope"]["hard_constraints"]
    assert all(evaluate(c, {"tile_m": 48, "tile_n": 40, "tile_k": 24}) for c in hard)
    assert all(evaluate(c, {"tile_m": 32, "tile_n": 16, "tile_k": 24}) for c in hard)
    assert not all(evaluate(c, {"tile_m": 64, "tile_n": 64, "tile_k": 24}) for c in hard)
    assert not all(evaluate(c, {"tile_m": 24, "tile_n": 32, "tile_k": 24}) for c in hard)
    assert not all(evaluate(c, {"tile_m": 48, "tile_n": 40, "tile_k": 25}) for c in hard)


@pytest.mark.parametrize("func", sorted(CASES))
def test_every_symbol_bounded_by_natural_ub(func):
    """Each symbol's natural_ub is an InRange bound of the scope: its value
    passes, natural_ub + 1 fails (the other symbols at a legal binding)."""
    syms, shapes = CASES[func]
    for dims in shapes:
        scope = loom_hip.constraint_scope(func, dims)["constraint_scope"]
        hard, meta = scope["hard_constraints"], scope["metadata"]["symbols"]
        pref = loom_hip.preferred_block_sizes(func, dims)
        for s in syms:
            ub = meta[s]["natural_ub"]
            assert {"InRange": {"x": {"Sym": s}, "lo": {"Const": 1}, "hi": {"Const": ub}}} in hard
            over = dict(pref, **{s: ub + 1})
            assert not all(evaluate(c, over) for c in hard), (func, dims, s)
            with pytest.raises(RuntimeError) as ei:
                loom_hip.check_variant(_variant(func, over), dims)
            assert ei.value.code == 1, (func, s, str(ei.value))


def test_hw_spec_is_the_scopes_machine_model():
    """loom_hip_hw_spec without a device: the LDS capacity is the one every
    footprint constraint uses, the built tiles are multiples of its tile
    alignment, and on large extents the values each tiled symbol takes in
    some legal binding are exactly the multiples of that alignment (each runs
    on the smallest listed tile covering it)."""
    spec = loom_hip.hw_spec()
    assert spec["target"] == "gfx950" and spec["wave_size"] == 64 and "device" not in spec
    big = {"matmul": (4096, 4096, 4096), "batch_matmul": (2, 4096, 4096, 4096),
           "split_k_matmul_gather": (4096, 4096, 16384), "attention": (128, 4096, 4096, 128),
           "helion_mamba2_chunk_scan_kernel": (4, 16, 32, 1, 256, 64, 128)}
    cand = sorted(set(GRID + [16, 32, 64, 128, 192, 256, 320, 512]))
    for func, dims in big.items():
        scope = loom_hip.constraint_scope(func, dims)["constraint_scope"]
        assert scope["metadata"]["capacity_bytes"] == spec["lds_bytes_per_workgroup"]
        syms = sorted(scope["metadata"]["symbols"])
        values = {s: (SMALL if s in ("tile_b", "tile_h", "tile_c") else cand) for s in syms}
        seen = {s: set() for s in syms}
        for combo in itertools.product(*(values[s] for s in syms)):
            env = dict(zip(syms, combo))
            if all(evaluate(c, env) for c in scope["hard_constraints"]):
                for s in syms:
                    seen[s].add(env[s])
        align = spec["tile_alignment"]
        for sym, built in spec["built_tiles"][func].items():
            assert all(t % align == 0 for t in built), (func, sym, built)
            ub = scope["metadata"]["symbols"][sym]["natural_ub"]
            want = [c for c in cand if c % align == 0 and c <= ub]
            assert sorted(seen[sym]) == want, (func, sym, sorted(seen[sym]), want)


def test_hw_spec_without_a_device_is_refused_cleanly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(RuntimeError) as ei:
        loom_hip.hw_spec(0)
    assert ei.value.code == 3 and "hw_spec" in str(ei.value)
