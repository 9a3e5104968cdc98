"""Synthetic workloads of the token-mixer benchmarks (seeded, host side).

Each generator returns numpy arrays; the same arrays feed the GPU path and
the CPU baseline / parity checks.  Streams are numpy PCG64 seeded with
(0x5EED0027 + config number, tag) so every input is reproducible.

  dn_recurrent   Gated DeltaNet recurrent decode without conv (q, k, v given;
                 q,k l2-normalised per head before the step, as the config
                 specifies)
  dn_conv        batched DeltaNet decode with the fused causal conv
  gqa_decode     gated GQA single-query decode over a bf16 KV cache
  dn_prefill_glue  a prompt through the whole DeltaNet branch of
                 vx27_qlayer_batch: projection outputs x, gates, z
"""
from __future__ import annotations

import zlib

import numpy as np

SEED = 0x5EED0027


def rng(config: int, tag: str):
    return np.random.default_rng([SEED + config, zlib.crc32(tag.encode())])


def normal(r, shape, std=1.0, mean=0.0):
    x = r.standard_normal(shape, dtype=np.float32)
    if std != 1.0:
        x *= np.float32(std)
    if mean != 0.0:
        x += np.float32(mean)
    return x


def l2norm_rows(x):
    """x * 1/sqrtf(sum x^2 + 1e-6) per last-axis row (the l2norm formula of
    vx27_deltanet.c:51-56; input preparation only)."""
    ss = np.sum(x.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(np.float32)
    inv = (np.float32(1.0) / np.sqrt(ss + np.float32(1e-6))).astype(np.float32)
    return (x * inv).astype(np.float32)


def bf16_bits(x):
    """Round-to-nearest-even bf16 bit patterns of float32 x."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(h):
    return (np.ascontiguousarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def dn_heads(r, nv):
    A_log = r.uniform(-2.0, 1.0, nv).astype(np.float32)
    dt_bias = normal(r, nv, 0.1)
    return A_log, dt_bias


def dn_recurrent(B=1, H=16, steps=2000, hd=128, config=1, S0_std=0.0):
    """Config: 16 heads, d_k = d_v = 128, fp32 state zero-init; per step q,k
    ~N(0,1) then l2-normalised per head, v ~N(0,1), beta = sigmoid(N(0,1)),
    a ~N(0,1); A_log ~U(-2,1), dt_bias ~N(0,0.1)."""
    r = rng(config, "dn_recurrent")
    A_log, dt_bias = dn_heads(r, H)
    d = dict(A_log=A_log, dt_bias=dt_bias)
    d["q"] = l2norm_rows(normal(r, (steps, B, H, hd)))
    d["k"] = l2norm_rows(normal(r, (steps, B, H, hd)))
    d["v"] = normal(r, (steps, B, H, hd))
    d["a"] = normal(r, (steps, B, H))
    d["b"] = normal(r, (steps, B, H))
    d["S0"] = (normal(r, (B, H, hd, hd), S0_std) if S0_std > 0
               else np.zeros((B, H, hd, hd), np.float32))
    return d


def dn_conv(B=64, H=16, steps=256, hd=128, config=3, S0_std=0.02, nv=None):
    """Config: batch B, H heads x 128x128 fp32 state ~N(0,0.02); causal conv
    width 4 with bf16 weights ~N(0,0.2) over the 3*H*128 q/k/v channels, then
    SiLU, l2norm q,k, q/sqrt(128), gates as dn_recurrent."""
    nv = nv or H
    r = rng(config, "dn_conv")
    C = 2 * H * hd + nv * hd
    A_log, dt_bias = dn_heads(r, nv)
    d = dict(A_log=A_log, dt_bias=dt_bias)
    d["conv_w_bf16"] = bf16_bits(normal(r, (C, 4), 0.2))
    d["conv_w"] = bf16_to_f32(d["conv_w_bf16"])
    d["conv0"] = np.zeros((B, C, 3), np.float32)
    d["S0"] = normal(r, (B, nv, hd, hd), S0_std)
    d["x"] = normal(r, (steps, B, C))
    d["a"] = normal(r, (steps, B, nv))
    d["b"] = normal(r, (steps, B, nv))
    return d


def dn_prefill(B=1, T=4096, nqk=16, nv=16, hd=128, config=4, S0_std=0.0):
    """Config: one prompt of T tokens; q,k,v ~N(0,1) stored bf16
    [B][T][heads][128] (q and k are l2-normalised inside, as step_exact does);
    a,b ~N(0,1) [B][T][nv]; A_log ~U(-2,1), dt_bias ~N(0,0.1); S0 zero."""
    r = rng(config, "dn_prefill")
    A_log, dt_bias = dn_heads(r, nv)
    d = dict(A_log=A_log, dt_bias=dt_bias)
    d["q"] = bf16_bits(normal(r, (B, T, nqk, hd)))
    d["k"] = bf16_bits(normal(r, (B, T, nqk, hd)))
    d["v"] = bf16_bits(normal(r, (B, T, nv, hd)))
    d["a"] = normal(r, (B, T, nv))
    d["b"] = normal(r, (B, T, nv))
    d["S0"] = (normal(r, (B, nv, hd, hd), S0_std) if S0_std > 0
               else np.zeros((B, nv, hd, hd), np.float32))
    return d


def dn_prefill_glue(B=1, T=4096, nqk=16, nv=48, hd=128, config=6, S0_std=0.02):
    """A prompt through the DeltaNet branch of vx27_qlayer_batch: the
    projection outputs x [B][T][C] (q|k|v channels, C = 2*nqk*hd + nv*hd),
    a, b [B][T][nv], z [B][T][nv][hd], all ~N(0,1); conv weights bf16
    ~N(0,0.2), conv state ~N(0,0.5), state ~N(0,0.02), norm weight
    1+N(0,0.1); A_log ~U(-2,1), dt_bias ~N(0,0.1)."""
    r = rng(config, "dn_prefill_glue")
    C = 2 * nqk * hd + nv * hd
    A_log, dt_bias = dn_heads(r, nv)
    d = dict(A_log=A_log, dt_bias=dt_bias)
    d["conv_w_bf16"] = bf16_bits(normal(r, (C, 4), 0.2))
    d["conv_w"] = bf16_to_f32(d["conv_w_bf16"])
    d["conv0"] = normal(r, (B, C, 3), 0.5)
    d["S0"] = normal(r, (B, nv, hd, hd), S0_std)
    d["norm_w"] = normal(r, hd, 0.1, 1.0)
    d["x"] = normal(r, (B, T, C))
    d["a"] = normal(r, (B, T, nv))
    d["b"] = normal(r, (B, T, nv))
    d["z"] = normal(r, (B, T, nv, hd))
    return d


def gqa_prefill(B=1, T=4096, n_q=24, n_kv=4, hd=256, pos0=0, config=5):
    """Config: one prompt of T tokens, bf16 ~N(0,1) raw q [B][T][24][256],
    gate logits [B][T][24][256], raw k, v [B][T][4][256]; q/k norm weights w
    with (1+w) ~ 1+N(0,0.1); RoPE at positions pos0..pos0+T-1; causal."""
    r = rng(config, "gqa_prefill")
    d = {"q": bf16_bits(normal(r, (B, T, n_q, hd))), "gate": bf16_bits(normal(r, (B, T, n_q, hd))),
         "k": bf16_bits(normal(r, (B, T, n_kv, hd))), "v": bf16_bits(normal(r, (B, T, n_kv, hd))),
         "q_norm_w": normal(r, hd, 0.1), "k_norm_w": normal(r, hd, 0.1), "pos0": pos0}
    return d


def gqa_decode(B=1, L=8192, n_q=24, n_kv=4, hd=256, config=2):
    """Config: bf16 KV cache of L positions with K,V ~N(0,1) (taken as already
    normed and roped), new token at position L; raw q ~N(0,1) and gate logits
    ~N(0,1) interleaved per head as q_proj emits them; k_new, v_new ~N(0,1);
    q/k norm weights w with (1+w) ~ 1+N(0,0.1)."""
    r = rng(config, f"gqa_decode_{B}_{L}")
    d = {}
    d["q_norm_w"] = normal(r, hd, 0.1)
    d["k_norm_w"] = normal(r, hd, 0.1)
    d["qg"] = normal(r, (B, n_q, 2 * hd))
    d["k_new"] = normal(r, (B, n_kv, hd))
    d["v_new"] = normal(r, (B, n_kv, hd))
    d["K"] = bf16_bits(normal(r, (B, L, n_kv, hd)))
    d["V"] = bf16_bits(normal(r, (B, L, n_kv, hd)))
    d["pos"] = np.full(B, L, np.int32)
    return d
