"""Writes the committed fixtures in this directory.

The reference commits no result vectors for this path, and its own oracles
(cuBLAS, the CUDA unfused attention) cannot run here. So the fixtures are
produced by routines independent of oracle/oracle.c:
  * sgemm_small.npz: inputs from the reference's xorshift fill
    (src/bench.cu:59-66, seeds bench.cu:226-228) re-implemented here in
    Python; C_f32seq by exact rational arithmetic with one rounding per fused
    multiply-add in k order; C_f64 by numpy.matmul in float64.
  * attention_small.npz: torch.nn.functional.scaled_dot_product_attention
    (is_causal=True) and torch.autograd in float64 on the CPU.
Run:  python tests/golden/make_golden.py
"""
import math
import os
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def xorshift_fill(n, seed):
    s = seed & 0xFFFFFFFF
    out = np.empty(n, np.float32)
    for i in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out[i] = np.float32((int(s % 2000) - 1000)) / np.float32(1000.0)
    return out


def round_f32(x):
    c = np.float32(float(x))
    cands = [np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))]
    return min(cands, key=lambda y: (abs(Fraction(float(y)) - x), int(np.float32(y).view(np.uint32)) & 1))


def fma32(a, b, c):
    return np.float32(round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))))


def sgemm_small():
    M, N, K = 13, 11, 17
    A = xorshift_fill(M * K, 0x12345678).reshape(M, K)
    B = xorshift_fill(K * N, 0x9ABCDEF0).reshape(K, N)
    C0 = xorshift_fill(M * N, 0x0F0F0F0F).reshape(M, N)
    alpha, beta = np.float32(0.5), np.float32(3.0)
    C = np.empty((M, N), np.float32)
    for i in range(M):
        for j in range(N):
            acc = np.float32(0.0)
            for k in range(K):
                acc = fma32(A[i, k], B[k, j], acc)
            C[i, j] = fma32(alpha, acc, np.float32(beta * C0[i, j]))
    C64 = 0.5 * (A.astype(np.float64) @ B.astype(np.float64)) + 3.0 * C0.astype(np.float64)
    np.savez(os.path.join(HERE, "sgemm_small.npz"), mnk=np.array([M, N, K]), A=A, B=B, C0=C0,
             C_f32seq=C, C_f64=C64)


def attention_small():
    import torch
    B, T, C, NH = 2, 7, 16, 2
    hs = C // NH
    rng = np.random.default_rng(20261201)
    qkv = rng.standard_normal((B, T, 3 * C)).astype(np.float32)
    dout = rng.standard_normal((B, T, C)).astype(np.float32)
    x = torch.from_numpy(qkv.astype(np.float64)).reshape(B, T, 3, NH, hs)
    q, k, v = (x[:, :, i].transpose(1, 2).clone().requires_grad_(True) for i in range(3))
    y = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True)
    s = (q @ k.transpose(-1, -2)) / math.sqrt(hs)
    lse = torch.logsumexp(s.masked_fill(~torch.ones(T, T, dtype=torch.bool).tril(), -math.inf), -1)
    g = torch.from_numpy(dout.astype(np.float64)).reshape(B, T, NH, hs).transpose(1, 2)
    grads = torch.autograd.grad(y, (q, k, v), g)
    dqkv = np.concatenate([t.transpose(1, 2).reshape(B, T, C).numpy() for t in grads], axis=2)
    np.savez(os.path.join(HERE, "attention_small.npz"), btcnh=np.array([B, T, C, NH]), qkv=qkv,
             dout=dout, out=y.transpose(1, 2).reshape(B, T, C).detach().numpy(),
             lse=lse.detach().numpy(), dqkv=dqkv)


if __name__ == "__main__":
    sgemm_small()
    attention_small()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
