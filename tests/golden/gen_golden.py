"""Writes the golden fixtures under tests/golden/ (run: python tests/golden/gen_golden.py).

The reference (loom-dataflow) ships no numeric tests, golden vectors or
known-answer data for any of the six kernels, and nothing of it can run here
(no MLIR toolchain).  These fixtures are therefore computed from textbook
definitions in float64 numpy, formulated independently of the oracle's
tiled / online algorithms:

  mm, bmm        : numpy matmul of the bf16-decoded inputs
  split-K        : integer-valued inputs, exact int64 per-slab products
  attention      : full (not online) softmax, optional causal mask
  flash_decode   : full softmax over the whole key range (no splits)
  mamba          : the sequential Mamba-2 recurrence
                       h_t = exp(dt_t A) h_{t-1} + dt_t B_t x_t^T
                       y_t = C_t h_t + D x_t
                   from the raw inputs (x, dt, A, B, C, D)

Each fixture holds its inputs (bf16 as raw uint16 bits) and the float64
expected output.  The inputs are seeded, so the files are reproducible.
"""
from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def to_bf16(a):
    f = np.ascontiguousarray(a, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def from_bf16(h):
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_normal(rng, shape, std=1.0):
    return to_bf16(rng.standard_normal(shape) * std)


def bf16_uniform(rng, shape, lo=-1.0, hi=1.0):
    return to_bf16(rng.uniform(lo, hi, shape))


def save(name, **arrays):
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)


# --------------------------------------------------------------------------
# fp64 textbook references
# --------------------------------------------------------------------------

def ref_matmul(x, y):
    return from_bf16(x).astype(np.float64) @ from_bf16(y).astype(np.float64)


def ref_attention(k, v, q, scale, causal):
    K = from_bf16(k).astype(np.float64)  # [BH, D, S]
    V = from_bf16(v).astype(np.float64)  # [BH, S, D]
    Qm = from_bf16(q).astype(np.float64)  # [BH, Sq, D]
    s = np.einsum("bid,bdj->bij", Qm, K) * scale
    if causal:
        sq, sk = s.shape[1], s.shape[2]
        mask = np.arange(sk)[None, :] > np.arange(sq)[:, None]
        s = np.where(mask[None], -np.inf, s)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("bij,bjd->bid", p, V)


def ref_decode(k, v, q, scale):
    # q [B,H,D] attends over all S keys of its batch: the same as attention
    # with Sq = H and no mask.
    return ref_attention(k, v, q, scale, causal=False)


def ref_mamba_recurrence(x, dt, A, Bm, Cm, Dh):
    """x [b,H,L,P] bf16; dt [b,H,L] f32; A [H]; B, C [b,G,L,N] bf16; D [H]."""
    X = from_bf16(x).astype(np.float64)
    Bf = from_bf16(Bm).astype(np.float64)
    Cf = from_bf16(Cm).astype(np.float64)
    dt = dt.astype(np.float64)
    b, H, L, P = X.shape
    G, N = Bf.shape[1], Bf.shape[3]
    hpg = H // G
    y = np.zeros((b, H, L, P))
    for bi in range(b):
        for h in range(H):
            g = h // hpg
            st = np.zeros((N, P))
            for t in range(L):
                st = np.exp(dt[bi, h, t] * A[h]) * st + dt[bi, h, t] * np.outer(Bf[bi, g, t], X[bi, h, t])
                y[bi, h, t] = Cf[bi, g, t] @ st + Dh[h] * X[bi, h, t]
    return y


# --------------------------------------------------------------------------
# fixtures
# --------------------------------------------------------------------------

def main():
    rng = np.random.default_rng(20261201)

    for name, (M, N, K) in {"mm_tiles": (128, 96, 160), "mm_ragged": (70, 50, 88)}.items():
        x = bf16_uniform(rng, (M, K))
        y = bf16_uniform(rng, (K, N))
        save(name, x=x, y=y, expected=ref_matmul(x, y))

    B, M, N, K = 3, 64, 96, 128
    a0 = bf16_normal(rng, (B, M, K), 0.5)
    a1 = bf16_normal(rng, (B, K, N), 0.5)
    save("bmm_small", arg0=a0, arg1=a1,
         expected=np.stack([ref_matmul(a0[i], a1[i]) for i in range(B)]))

    # split-K with small integers: every partial and the sum are exact in fp32
    M, N, K, tk = 64, 96, 1024, 128
    ai = rng.integers(-4, 5, (M, K))
    bi = rng.integers(-4, 5, (K, N))
    S = K // tk
    parts = np.stack([ai[:, s * tk:(s + 1) * tk] @ bi[s * tk:(s + 1) * tk, :] for s in range(S)])
    save("splitk_int", a=to_bf16(ai), b=to_bf16(bi), tile_k=np.int64(tk),
         expected_partials=parts.astype(np.float64), expected=parts.sum(0).astype(np.float64))

    M, N, K, tk = 48, 64, 768, 256
    a = bf16_normal(rng, (M, K), 0.1)
    b = bf16_normal(rng, (K, N), 0.1)
    save("splitk_float", a=a, b=b, tile_k=np.int64(tk), expected=ref_matmul(a, b))

    for name, (BH, S, D, causal) in {
        "attention_noncausal": (2, 96, 64, False),
        "attention_causal": (2, 80, 128, True),
    }.items():
        k = bf16_normal(rng, (BH, D, S))
        v = bf16_normal(rng, (BH, S, D))
        q = bf16_normal(rng, (BH, S, D))
        scale = 1.0 / np.sqrt(D)
        save(name, k=k, v=v, q=q, scale=np.float64(scale), causal=np.int64(causal),
             expected=ref_attention(k, v, q, scale, causal))

    for name, (B, H, D, S) in {"decode_ragged": (2, 8, 64, 200), "decode_mqa": (2, 32, 128, 512)}.items():
        k = bf16_normal(rng, (B, D, S))
        v = bf16_normal(rng, (B, S, D))
        q = bf16_normal(rng, (B, H, D))
        scale = 1.0 / np.sqrt(D)
        save(name, k=k, v=v, q=q, scale=np.float64(scale), expected=ref_decode(k, v, q, scale))

    b, H, G, L, P, N, Q = 1, 4, 2, 64, 16, 16, 16
    x = bf16_normal(rng, (b, H, L, P))
    Bm = bf16_normal(rng, (b, G, L, N))
    Cm = bf16_normal(rng, (b, G, L, N))
    dt = np.log1p(np.exp(rng.standard_normal((b, H, L)))).astype(np.float32)
    A = (-np.exp(rng.uniform(0.0, 1.0, H))).astype(np.float32)
    Dh = rng.standard_normal(H).astype(np.float32)
    save("mamba_small", x=x, dt=dt, A=A, B=Bm, C=Cm, D=Dh, chunk_size=np.int64(Q),
         expected=ref_mamba_recurrence(x, dt, A, Bm, Cm, Dh))


if __name__ == "__main__":
    main()
