import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "loom-dataflow_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_golden(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture
def golden():
    return load_golden


# every tolerance check of the run: (what, elements, max |err|, max |err|/|ref|
# over |ref| >= atol, largest err / (atol + rtol |ref|)), printed at the end
ERRORS = []


def _record(what, n, max_abs, max_rel, used):
    ERRORS.append((what, n, max_abs, max_rel, used))


def assert_close(actual, expected, atol, rtol, what=""):
    """|actual - expected| <= atol + rtol * |expected| elementwise (NaN fails)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, (a.shape, e.shape)
    err = np.abs(a - e)
    bound = atol + rtol * np.abs(e)
    bad = ~(err <= bound)
    if bad.any():
        idx = np.unravel_index(np.argmax(np.where(bad, err - bound, -np.inf)), a.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{a.size} elements outside atol={atol} rtol={rtol}; "
            f"worst at {idx}: got {a[idx]!r} expected {e[idx]!r}; max abs err {err.max():.3e}")
    if a.size:
        big = np.abs(e) >= atol
        _record(what, a.size, float(err.max()),
                float((err[big] / np.abs(e[big])).max()) if big.any() else 0.0,
                float((err / bound).max()))


def assert_close_gpu(actual, expected, atol, rtol, what=""):
    """assert_close for torch tensors on the GPU (full BASELINE-size outputs,
    too large to copy and compare in numpy): compared in fp32 there."""
    import torch
    a, e = actual.float(), expected.float()
    assert a.shape == e.shape, (tuple(a.shape), tuple(e.shape))
    err = (a - e).abs()
    bound = atol + rtol * e.abs()
    bad = ~(err <= bound)
    nbad = int(bad.sum())
    if nbad:
        i = int(torch.argmax(torch.where(bad, err, torch.zeros_like(err))))
        raise AssertionError(
            f"{what}: {nbad}/{a.numel()} elements outside atol={atol} rtol={rtol}; worst at flat "
            f"index {i}: got {float(a.flatten()[i])!r} expected {float(e.flatten()[i])!r}")
    if a.numel():
        big = e.abs() >= atol
        rel = float((err[big] / e.abs()[big]).max()) if bool(big.any()) else 0.0
        _record(what, a.numel(), float(err.max()), rel, float((err / bound).max()))


def pytest_terminal_summary(terminalreporter):
    """The error margins of every tolerance check that passed: max abs and
    max rel error against the reference, and the largest share of the
    tolerance any element used."""
    # pytest loads this file as `conftest`, the tests import it as
    # `tests.conftest`: two module objects, each with its own list
    mods = {id(m): m for m in (sys.modules.get("conftest"), sys.modules.get("tests.conftest"))
            if m is not None and hasattr(m, "ERRORS")}
    errors = [e for m in mods.values() for e in m.ERRORS]
    if not errors:
        return
    tr = terminalreporter
    tr.section("tolerance checks (max abs err, max rel err where |ref| >= atol, share of tolerance used)")
    for what, n, ma, mr, used in errors:
        tr.write_line(f"{what[:60]:60s} {n:>10d}  {ma:10.3e}  {mr:10.3e}  {used:6.3f}")


GEMM_TILES = (64, 128, 256)
ATTN_TILES = (64, 128, 192, 256)
MAMBA_M_TILES = (64, 128, 192, 256)
MAMBA_N_TILES = (16, 32, 64)


def tile_for(T, extent, built):
    """The tile_* value that makes a kernel run workgroup tile T along an axis
    of `extent`: T itself within the extent (every symbol is bounded by its
    loop extent, natural_ub), the whole extent when T is the smallest built
    tile covering it, else None (T cannot be bound for this extent)."""
    if T <= extent:
        return T
    cover = [t for t in built if t >= extent]
    return extent if cover and min(cover) == T else None
