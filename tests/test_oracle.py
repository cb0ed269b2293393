"""Pins the fp32 CPU oracle (oracle/oracle.c) before it is trusted as the checker.

The reference ships no golden vectors or known-answer tests, so each oracle
function is pinned by checks that do not retype its formula:

  matmul / batch_matmul
      float64 numpy matmul fixtures (tests/golden/mm_*.npz, bmm_small.npz);
      identity and permutation right operands (out == x exactly);
      integer-valued inputs (exact); bitwise invariance to the tile sizes.
  split_k_matmul_gather
      integer-valued inputs: every K-slab partial G[s] and the output equal
      exact int64 slab products (splitk_int.npz); float fixture; invariance
      to the split count.
  attention
      full-softmax float64 fixtures, causal and not (attention_*.npz);
      identical V rows -> out == that row; Q = 0 -> mean of V (causal:
      prefix mean); one dominant logit -> its V row; invariance to tile_n.
  flash_decode
      full-softmax float64 fixtures (decode_*.npz); each split's lse_s and
      o_s against float64 logsumexp / softmax over that split alone;
      invariance to the split size.
  mamba_prologue + mamba_chunk_scan
      the whole chain against the sequential SSM recurrence in float64
      (mamba_small.npz); dA_cumsum against numpy cumsum; cb against numpy
      C B^T (masked); prev_states_T against the recurrence's state at each
      chunk boundary; C = 0 -> out == bf16(D x) exactly; invariance to
      tile_k.
"""
import numpy as np
import pytest

import oracle
from oracle import from_bf16, to_bf16
from tests.conftest import assert_close

RT = 2.0 ** -8 * 1.01  # one bf16 rounding of the output


# ----------------------------------------------------------------------- mm

@pytest.mark.parametrize("name", ["mm_tiles", "mm_ragged"])
def test_matmul_golden(golden, name):
    g = golden(name)
    out = oracle.matmul(g["x"], g["y"], 32, 32, 32)
    assert_close(from_bf16(out), g["expected"], atol=1e-4, rtol=RT, what=name)


def test_matmul_identity_and_permutation():
    rng = np.random.default_rng(1)
    x = to_bf16(rng.standard_normal((96, 64)))
    eye = to_bf16(np.eye(64))
    assert np.array_equal(oracle.matmul(x, eye, 32, 32, 16), x)
    perm = rng.permutation(64)
    pm = to_bf16(np.eye(64)[:, perm])
    assert np.array_equal(oracle.matmul(x, pm, 64, 64, 64), x[:, perm])


def test_matmul_integer_exact_and_tile_invariant():
    rng = np.random.default_rng(2)
    xi = rng.integers(-8, 9, (80, 144))
    yi = rng.integers(-8, 9, (144, 112))
    ref = xi @ yi  # |ref| < 2^14: exact in bf16 only if representable; compare via fp32
    outs = [oracle.matmul(to_bf16(xi), to_bf16(yi), *t) for t in
            [(16, 16, 16), (80, 112, 144), (32, 64, 48), (7, 9, 11)]]
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])
    assert np.array_equal(outs[0], to_bf16(ref.astype(np.float32)))


def test_matmul_rejects_bad_tiles():
    x = to_bf16(np.ones((8, 8)))
    with pytest.raises(ValueError):
        oracle.split_k_matmul_gather(x, x, 8, 8, 9)  # tile_k > K
    with pytest.raises(ValueError):
        oracle.matmul(x, x, 0, 8, 8)


def test_batch_matmul_golden(golden):
    g = golden("bmm_small")
    out = oracle.batch_matmul(g["arg0"], g["arg1"], 1, 32, 32, 32)
    assert_close(from_bf16(out), g["expected"], atol=1e-4, rtol=RT, what="bmm")
    for b in range(out.shape[0]):
        assert np.array_equal(out[b], oracle.matmul(g["arg0"][b], g["arg1"][b], 64, 64, 64))


# ------------------------------------------------------------------ split-K

def test_split_k_integer_partials_exact(golden):
    g = golden("splitk_int")
    out, parts = oracle.split_k_matmul_gather(g["a"], g["b"], 32, 32, int(g["tile_k"]))
    assert parts.shape == g["expected_partials"].shape
    assert np.array_equal(parts.astype(np.float64), g["expected_partials"])
    assert np.array_equal(out, to_bf16(g["expected"].astype(np.float32)))


def test_split_k_float_and_split_invariance(golden):
    g = golden("splitk_float")
    out, parts = oracle.split_k_matmul_gather(g["a"], g["b"], 16, 32, int(g["tile_k"]))
    assert parts.shape[0] == 768 // 256
    assert_close(from_bf16(out), g["expected"], atol=1e-4, rtol=RT, what="splitk")
    out2, parts2 = oracle.split_k_matmul_gather(g["a"], g["b"], 48, 64, 768)
    assert parts2.shape[0] == 1
    assert_close(from_bf16(out2), from_bf16(out), atol=1e-4, rtol=2 * RT, what="S=1 vs S=3")
    # a ragged last slab: K = 768 with tile_k = 500 -> slabs of 500 and 268
    out3, parts3 = oracle.split_k_matmul_gather(g["a"], g["b"], 16, 16, 500)
    assert parts3.shape[0] == 2
    assert_close(parts3.sum(0), from_bf16(out).astype(np.float64), atol=1e-3, rtol=2 * RT,
                 what="ragged slabs")


# ---------------------------------------------------------------- attention

@pytest.mark.parametrize("name", ["attention_noncausal", "attention_causal"])
def test_attention_golden(golden, name):
    g = golden(name)
    out = oracle.attention(g["k"], g["v"], g["q"], float(g["scale"]), bool(g["causal"]),
                           1, 32, 32)
    assert_close(from_bf16(out), g["expected"], atol=1e-3, rtol=RT, what=name)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_tile_n_invariance(golden, causal):
    g = golden("attention_causal")
    args = (g["k"], g["v"], g["q"], float(g["scale"]), causal)
    ref = from_bf16(oracle.attention(*args, 1, 80, 80))
    for tm, tn in [(16, 16), (32, 48), (64, 7)]:
        o = from_bf16(oracle.attention(*args, 1, tm, tn))
        assert_close(o, ref, atol=1e-3, rtol=2 * RT, what=f"tiles {tm},{tn}")


def test_attention_closed_forms():
    rng = np.random.default_rng(3)
    BH, S, D = 2, 40, 16
    q = to_bf16(rng.standard_normal((BH, S, D)))
    k = to_bf16(rng.standard_normal((BH, D, S)))
    # identical V rows -> every output row is that row, for any weights
    row = to_bf16(rng.standard_normal(D))
    v_same = np.broadcast_to(row, (BH, S, D)).copy()
    for causal in (False, True):
        out = oracle.attention(k, v_same, q, 0.25, causal, 1, 16, 16)
        assert np.array_equal(out, np.broadcast_to(row, out.shape))
    # Q = 0 -> uniform weights: mean of V (causal: running prefix mean)
    v = to_bf16(rng.standard_normal((BH, S, D)))
    zeros = np.zeros((BH, S, D), np.uint16)
    vf = from_bf16(v).astype(np.float64)
    out = oracle.attention(k, v, zeros, 0.125, False, 1, 16, 16)
    assert_close(from_bf16(out), np.broadcast_to(vf.mean(1, keepdims=True), vf.shape),
                 atol=1e-5, rtol=RT, what="Q=0")
    out = oracle.attention(k, v, zeros, 0.125, True, 1, 16, 16)
    prefix = np.cumsum(vf, axis=1) / np.arange(1, S + 1)[None, :, None]
    assert_close(from_bf16(out), prefix, atol=1e-5, rtol=RT, what="Q=0 causal")
    # one dominant logit: key j* gets score 100*scale*|q|^2 -> output is v[j*]
    qd = np.zeros((1, 4, D), np.float32)
    qd[0, :, 0] = 4.0
    kd = np.zeros((1, D, 12), np.float32)
    kd[0, 0, 5] = 30.0
    vd = rng.standard_normal((1, 12, D)).astype(np.float32)
    out = oracle.attention(to_bf16(kd), to_bf16(vd), to_bf16(qd), 1.0, False, 1, 4, 4)
    assert np.array_equal(out[0], np.broadcast_to(to_bf16(vd[0, 5]), (4, D)))


# ------------------------------------------------------------- flash_decode

@pytest.mark.parametrize("name,tile_s,tile_n", [("decode_ragged", 64, 16),
                                                ("decode_ragged", 200, 200),
                                                ("decode_mqa", 128, 64)])
def test_decode_golden(golden, name, tile_s, tile_n):
    g = golden(name)
    out, lse, o = oracle.flash_decode(g["k"], g["v"], g["q"], float(g["scale"]), 1, tile_s, tile_n)
    assert_close(from_bf16(out), g["expected"], atol=1e-3, rtol=RT, what=name)


def test_decode_split_partials(golden):
    """lse_s and o_s of every split against float64 softmax over that split only."""
    g = golden("decode_ragged")
    scale = float(g["scale"])
    tile_s = 64
    out, lse, o = oracle.flash_decode(g["k"], g["v"], g["q"], scale, 1, tile_s, 32)
    K = from_bf16(g["k"]).astype(np.float64)
    V = from_bf16(g["v"]).astype(np.float64)
    Qh = from_bf16(g["q"]).astype(np.float64)
    S = K.shape[2]
    ns = -(-S // tile_s)
    assert lse.shape == (ns,) + Qh.shape[:2]
    for s in range(ns):
        sl = slice(s * tile_s, min(S, (s + 1) * tile_s))
        sc = np.einsum("bhd,bdn->bhn", Qh, K[:, :, sl]) * scale
        mx = sc.max(-1, keepdims=True)
        lse_ref = np.log(np.exp(sc - mx).sum(-1)) + mx[..., 0]
        p = np.exp(sc - lse_ref[..., None])
        o_ref = np.einsum("bhn,bnd->bhd", p, V[:, sl])
        assert_close(lse[s], lse_ref, atol=1e-4, rtol=1e-5, what=f"lse split {s}")
        assert_close(o[s], o_ref, atol=1e-4, rtol=1e-4, what=f"o split {s}")


# -------------------------------------------------------------------- mamba

def _mamba_chain(g, tiles=(16, 16, 16)):
    Q = int(g["chunk_size"])
    dt, dA, cb, prev = oracle.mamba_prologue(g["x"], g["dt"], g["A"], g["B"], g["C"], Q)
    out = oracle.mamba_chunk_scan(cb, g["x"], dt, dA, g["C"], g["D"], prev, *tiles)
    return out, (dt, dA, cb, prev)


def test_mamba_chain_matches_recurrence(golden):
    g = golden("mamba_small")
    out, _ = _mamba_chain(g)
    # tolerance covers the bf16 rounding of cb (|cb| ~ sqrt(N)) and of the output
    assert_close(from_bf16(out), g["expected"], atol=2e-2, rtol=1e-2, what="mamba chain")


def test_mamba_prologue_pieces(golden):
    g = golden("mamba_small")
    Q = int(g["chunk_size"])
    _, (dt, dA, cb, prev) = _mamba_chain(g)
    x = from_bf16(g["x"]).astype(np.float64)
    Bf = from_bf16(g["B"]).astype(np.float64)
    Cf = from_bf16(g["C"]).astype(np.float64)
    b, H, L, P = x.shape
    G, N = Bf.shape[1], Bf.shape[3]
    nc = L // Q
    dtc = g["dt"].astype(np.float64).reshape(b, H, nc, Q)
    assert np.array_equal(dt, g["dt"].reshape(b, H, nc, Q))
    assert_close(dA, np.cumsum(dtc * g["A"].astype(np.float64)[None, :, None, None], -1),
                 atol=1e-5, rtol=1e-5, what="dA_cumsum")
    Cc = Cf.reshape(b, G, nc, Q, N)
    Bc = Bf.reshape(b, G, nc, Q, N)
    cb_ref = np.einsum("bgcmn,bgckn->bcgmk", Cc, Bc) * np.tril(np.ones((Q, Q)))
    assert_close(from_bf16(cb), cb_ref, atol=1e-5, rtol=RT, what="cb")
    # prev_states_T[b, c] == recurrence state after position c*Q - 1
    A = g["A"].astype(np.float64)
    dtf = g["dt"].astype(np.float64)
    hpg = H // G
    for bi in range(b):
        for h in range(H):
            st = np.zeros((N, P))
            for t in range(L):
                if t % Q == 0:
                    assert_close(prev[bi, t // Q, h], st, atol=1e-4, rtol=1e-4,
                                 what=f"prev b{bi} h{h} c{t // Q}")
                st = np.exp(dtf[bi, h, t] * A[h]) * st + dtf[bi, h, t] * np.outer(
                    Bf[bi, h // hpg, t], x[bi, h, t])


def test_mamba_c_zero_is_skip_connection(golden):
    g = dict(golden("mamba_small"))
    g["C"] = np.zeros_like(g["C"])
    out, _ = _mamba_chain(g)
    xf = from_bf16(g["x"])
    expect = to_bf16(xf * g["D"][None, :, None, None])
    assert np.array_equal(out, expect)


def test_mamba_tile_invariance(golden):
    g = golden("mamba_small")
    ref, _ = _mamba_chain(g, (16, 16, 16))
    for t in [(4, 8, 4), (16, 16, 3), (8, 5, 32)]:
        o, _ = _mamba_chain(g, t)
        assert_close(from_bf16(o), from_bf16(ref), atol=1e-3, rtol=2 * RT, what=str(t))


# ------------------------------------------------------------- f16 element mode
# The oracle's f16 conversions are written from the IEEE 754 binary16 layout;
# numpy's float16 (an independent implementation) pins them: every one of the
# 65536 patterns widens identically, and rounding agrees on every float32
# class -- normals, the subnormal range and its boundary, halfway cases,
# overflow to infinity at 65520, zeros, infinities and NaN.

def test_f16_widen_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    with oracle.element_type("f16"):
        got = oracle.widen16(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


@pytest.mark.filterwarnings("ignore::RuntimeWarning")
def test_f16_round_matches_numpy():
    rng = np.random.default_rng(5)
    parts = [
        (rng.standard_normal(200000) * 10.0 ** rng.integers(-9, 6, 200000)).astype(np.float32),
        rng.uniform(-70000, 70000, 100000).astype(np.float32),
        # halfway points between consecutive f16 values, normal and subnormal
        (np.arange(0, 65535, dtype=np.uint32).astype(np.uint16).view(np.float16)
         .astype(np.float64)[:-1] + np.diff(np.arange(0, 65535, dtype=np.uint32).astype(np.uint16)
                                             .view(np.float16).astype(np.float64)) / 2)
        .astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, -65520.0, 2.0 ** -14, 2.0 ** -24,
                  2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -26, np.inf, -np.inf], np.float32),
    ]
    with np.errstate(invalid="ignore", over="ignore"):
        x = np.concatenate([p[np.isfinite(p)] for p in parts[:3]] + [parts[3]]).astype(np.float32)
    with oracle.element_type("f16"):
        got = oracle.round16(x)
    ref = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, ref)
    with oracle.element_type("f16"):
        assert np.isnan(oracle.round16(np.array([np.nan], np.float32)).view(np.float16)[0])


def test_element_type_is_scoped():
    x = np.array([1.0 / 3.0], np.float32)
    with oracle.element_type("f16"):
        assert oracle.round16(x)[0] == np.float16(1 / 3).view(np.uint16)
    assert oracle.round16(x)[0] == oracle.to_bf16(x)[0]


def test_f16_matmul_and_attention_against_float64():
    """The restated functions in f16 mode: inputs widen from f16, outputs
    round to f16 (checked against float64 brute force of the same f16 values)."""
    rng = np.random.default_rng(6)
    x = oracle.to_f16(rng.standard_normal((40, 72)))
    y = oracle.to_f16(rng.standard_normal((72, 24)))
    with oracle.element_type("f16"):
        out = oracle.from_f16(oracle.matmul(x, y, 16, 16, 32))
    ref = oracle.from_f16(x).astype(np.float64) @ oracle.from_f16(y).astype(np.float64)
    np.testing.assert_allclose(out, ref, rtol=2e-3, atol=2e-3)
    # integer-valued operands: every product and sum exact, one rounding
    xi = oracle.to_f16(rng.integers(-4, 5, (32, 64)).astype(np.float32))
    yi = oracle.to_f16(rng.integers(-4, 5, (64, 16)).astype(np.float32))
    with oracle.element_type("f16"):
        oi = oracle.matmul(xi, yi, 16, 16, 16)
    exact = oracle.from_f16(xi).astype(np.int64) @ oracle.from_f16(yi).astype(np.int64)
    np.testing.assert_array_equal(oi, oracle.to_f16(exact.astype(np.float32)))
    BH, S, D = 2, 48, 32
    k = oracle.to_f16(rng.standard_normal((BH, D, S)))
    v = oracle.to_f16(rng.standard_normal((BH, S, D)))
    q = oracle.to_f16(rng.standard_normal((BH, S, D)))
    with oracle.element_type("f16"):
        o = oracle.from_f16(oracle.attention(k, v, q, 1 / np.sqrt(D), True, 1, 16, 16))
    kf, vf, qf = (oracle.from_f16(t).astype(np.float64) for t in (k, v, q))
    s = np.einsum("bqd,bdk->bqk", qf, kf) / np.sqrt(D)
    s[:, np.triu_indices(S, 1)[0], np.triu_indices(S, 1)[1]] = -np.inf
    p = np.exp(s - s.max(-1, keepdims=True))
    ref = np.einsum("bqk,bkd->bqd", p / p.sum(-1, keepdims=True), vf)
    np.testing.assert_allclose(o, ref, rtol=2e-3, atol=2e-3)
