"""Seeded synthetic inputs for the mla-moe hot path (DeepSeek-V2-Lite shapes).

Weights are bf16 stored as uint16, produced from float32 N(0, std) samples by
truncation, which is the reference's own fp32 -> bf16 rule (include/tensor.h:16-20).
Activations are float32 N(0, 1).  The generator is numpy's PCG64
`default_rng(seed)`, so host-side inputs are identical on every machine that
runs this image.
"""
from __future__ import annotations

import numpy as np

# DeepSeek-V2-Lite MoE / MLA geometry.
DSV2 = dict(H=2048, E=64, K=6, I=1408, n_shared=2, NH=16, QKN=128, QKR=64, KVL=512, VHD=128)


def bf16_from_f32(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 by truncation (include/tensor.h:16-20)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    return (a.view(np.uint32) >> 16).astype(np.uint16)


def bf16_to_f32(u: np.ndarray) -> np.ndarray:
    """bf16 -> fp32 by a 16-bit shift (include/tensor.h:9-14)."""
    u = np.ascontiguousarray(u, dtype=np.uint16)
    return (u.astype(np.uint32) << 16).view(np.float32)


def normal_f32(rng: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    x = rng.standard_normal(size=shape, dtype=np.float32)
    if std != 1.0:
        x *= np.float32(std)
    return x


def normal_bf16(rng: np.random.Generator, shape, std: float = 0.02) -> np.ndarray:
    return bf16_from_f32(normal_f32(rng, shape, std))


def moe_layer(seed: int, H: int, E: int, I: int, n_shared: int, std: float = 0.02,
              gate_bias: bool = False) -> dict:
    """One MoE layer's bf16 weights: router [E,H], experts gate/up [E,I,H],
    down [E,H,I], shared gate/up [S,H], down [H,S] with S = n_shared*I."""
    rng = np.random.default_rng(seed)
    S = n_shared * I
    w = dict(
        moe_gate=normal_bf16(rng, (E, H), std),
        eg=normal_bf16(rng, (E, I, H), std),
        eu=normal_bf16(rng, (E, I, H), std),
        ed=normal_bf16(rng, (E, H, I), std),
        sg=normal_bf16(rng, (S, H), std),
        su=normal_bf16(rng, (S, H), std),
        sd=normal_bf16(rng, (H, S), std),
    )
    w["moe_gate_bias"] = normal_f32(rng, (E,), 0.1) if gate_bias else None
    return w


def attn_layer(seed: int, H: int, NH: int, QKN: int, QKR: int, KVL: int, VHD: int,
               q_lora: int = 0, std: float = 0.02) -> dict:
    """One MLA layer's bf16 weights (nn.Linear layout [out, in]): the
    input_layernorm, q_proj [NH*(QKN+QKR), H] (or, with q_lora > 0, q_a_proj
    [q_lora, H], q_a_layernorm and q_b_proj [NH*(QKN+QKR), q_lora]),
    kv_a_proj [KVL+QKR, H], kv_a_layernorm, the head-interleaved kv_b
    [NH*(QKN+VHD), KVL] and o_proj [H, NH*VHD].  Norm weights are
    1 + N(0, 0.1) so that a dropped norm multiply shows."""
    rng = np.random.default_rng(seed)
    QD = NH * (QKN + QKR)

    def norm(n):
        return bf16_from_f32(1.0 + normal_f32(rng, (n,), 0.1))

    w = dict(in_norm=norm(H), q_proj=None, q_a_proj=None, q_a_norm=None, q_b_proj=None)
    if q_lora > 0:
        w.update(q_a_proj=normal_bf16(rng, (q_lora, H), std), q_a_norm=norm(q_lora),
                 q_b_proj=normal_bf16(rng, (QD, q_lora), std))
    else:
        w["q_proj"] = normal_bf16(rng, (QD, H), std)
    w.update(kv_a=normal_bf16(rng, (KVL + QKR, H), std), kv_a_norm=norm(KVL),
             kv_b=normal_bf16(rng, (NH * (QKN + VHD), KVL), std),
             o_proj=normal_bf16(rng, (H, NH * VHD), std))
    return w


def model(seed: int, n_layers: int, first_dense: int, H: int, NH: int, QKN: int, QKR: int,
          KVL: int, VHD: int, dense_inter: int, E: int, I: int, n_shared: int, vocab: int,
          gate_bias: bool = False, q_lora: int = 0) -> dict:
    """A whole decoder's bf16 weights with DeepSeek-V2's layout: embed
    [vocab, H], per layer an attn_layer() dict plus post_norm and either a
    dense MLP (dgate/dup [dense_inter, H], ddown [H, dense_inter]) for the
    first `first_dense` layers or a moe_layer() dict, then the final norm and
    lm_head [vocab, H].  Layer l's tensors come from seed + 100 (l + 1)."""
    rng = np.random.default_rng(seed)
    m = dict(embed=normal_bf16(rng, (vocab, H), 1.0),
             final_norm=bf16_from_f32(1.0 + normal_f32(rng, (H,), 0.1)),
             lm_head=normal_bf16(rng, (vocab, H), 0.02), layers=[])
    for l in range(n_layers):
        s = seed + 100 * (l + 1)
        lw = attn_layer(s, H, NH, QKN, QKR, KVL, VHD, q_lora)
        r = np.random.default_rng(s + 1)
        lw["post_norm"] = bf16_from_f32(1.0 + normal_f32(r, (H,), 0.1))
        if l < first_dense:
            lw.update(dgate=normal_bf16(r, (dense_inter, H)), dup=normal_bf16(r, (dense_inter, H)),
                      ddown=normal_bf16(r, (H, dense_inter)))
        else:
            lw.update(moe_layer(s + 2, H, E, I, n_shared, gate_bias=gate_bias))
        m["layers"].append(lw)
    return m


def activations(seed: int, T: int, H: int) -> np.ndarray:
    return normal_f32(np.random.default_rng(seed), (T, H))


def zipf_prior(seed: int, E: int, s: float = 1.1) -> np.ndarray:
    """Per-expert logit prior z_e = -s * ln(1 + pi(e)), pi a seeded permutation:
    expert pi^-1(r) gets the prior of Zipf rank r+1, which skews the load."""
    perm = np.random.default_rng(seed).permutation(E)
    return (-np.float64(s) * np.log1p(perm.astype(np.float64))).astype(np.float32)


def uniform_logits(seed: int, T: int, E: int) -> np.ndarray:
    return np.random.default_rng(seed).random((T, E), dtype=np.float32)


def checksum_u16(a: np.ndarray) -> int:
    """Order-sensitive 64-bit checksum of a uint16 array, used to assert that a
    regenerated weight tensor equals the one a golden vector was made from."""
    v = np.ascontiguousarray(a, dtype=np.uint16).ravel().astype(np.uint64)
    pos = np.arange(v.size, dtype=np.uint64)
    return int((v * (pos % np.uint64(65521) + np.uint64(1))).sum(dtype=np.uint64))
