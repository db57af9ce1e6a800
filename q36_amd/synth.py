"""Seeded synthetic inputs for the W4A8 MoE layer (numpy, host side).

Distributions follow the benchmark configurations of the q36 MoE layer:
MXFP4 weights with E2M1 codes uniform over the 16 values and one E8M0 scale
per 32 elements with exponent uniform in [-8, 0]; activations and router
logits N(0, 1); Zipf(s)-skewed routing for ragged batches.

Weights are produced in the GGUF block_mxfp4 format (17-byte blocks: E8M0
byte then 16 bytes of nibbles, q36.h:112-114) so they enter the library
through the same upload path as a real model file.
"""
import numpy as np

D_MODEL = 2048
N_EXPERT = 256
D_FF = 512
TOP_K = 8


def mxfp4_blocks(rng, rows, k, exp_lo=-8, exp_hi=0):
    """[rows, k/32, 17] uint8 GGUF MXFP4 blocks."""
    nb = k // 32
    blk = np.frombuffer(rng.bytes(rows * nb * 17), dtype=np.uint8).reshape(rows, nb, 17).copy()
    blk[:, :, 0] = (127 + rng.integers(exp_lo, exp_hi + 1, size=(rows, nb))).astype(np.uint8)
    return blk


def expert_weights(seed, n_expert=N_EXPERT, d_model=D_MODEL, d_ff=D_FF, shared=False):
    """dict gate/up [E, d_ff, d_model/32, 17], down [E, d_model, d_ff/32, 17]
    and, if shared, sh_gate/sh_up [d_ff, d_model/32, 17], sh_down."""
    rng = np.random.default_rng(seed)
    w = {
        "gate": mxfp4_blocks(rng, n_expert * d_ff, d_model).reshape(n_expert, d_ff, d_model // 32, 17),
        "up": mxfp4_blocks(rng, n_expert * d_ff, d_model).reshape(n_expert, d_ff, d_model // 32, 17),
        "down": mxfp4_blocks(rng, n_expert * d_model, d_ff).reshape(n_expert, d_model, d_ff // 32, 17),
    }
    if shared:
        w["sh_gate"] = mxfp4_blocks(rng, d_ff, d_model).reshape(d_ff, d_model // 32, 17)
        w["sh_up"] = mxfp4_blocks(rng, d_ff, d_model).reshape(d_ff, d_model // 32, 17)
        w["sh_down"] = mxfp4_blocks(rng, d_model, d_ff).reshape(d_model, d_ff // 32, 17)
    return w


GGML_Q8_0, GGML_Q5_K, GGML_Q6_K = 8, 13, 14
KQUANT_BLOCK = {GGML_Q8_0: (32, 34), GGML_Q5_K: (256, 176), GGML_Q6_K: (256, 210)}


def _f16_bytes(rng, n, lo, hi):
    return np.frombuffer(rng.uniform(lo, hi, size=n).astype(np.float16).tobytes(), dtype=np.uint8).reshape(n, 2)


def kquant_blocks(rng, rows, k, ggml_type):
    """[rows, row bytes] uint8 GGUF blocks of a Q8_0 / Q5_K / Q6_K matrix with
    random codes and finite f16 super-block scales (the formats of the
    reference's fallback expert tensors, q36.h:109-131), sized so values
    span roughly the MXFP4 experts' range."""
    elems, size = KQUANT_BLOCK[ggml_type]
    nb = rows * (k // elems)
    blk = np.frombuffer(rng.bytes(nb * size), dtype=np.uint8).reshape(nb, size).copy()
    if ggml_type == GGML_Q8_0:
        blk[:, 0:2] = _f16_bytes(rng, nb, 0.005, 0.05)
    elif ggml_type == GGML_Q5_K:
        blk[:, 0:2] = _f16_bytes(rng, nb, 5e-4, 3e-3)      # d
        blk[:, 2:4] = _f16_bytes(rng, nb, 5e-4, 3e-3)      # dmin
    else:
        blk[:, 208:210] = _f16_bytes(rng, nb, 5e-4, 3e-3)  # d
    return blk.reshape(rows, -1)


def hidden(rng, T, d_model=D_MODEL):
    return rng.standard_normal((T, d_model), dtype=np.float32)


def normal_logits(rng, T, n_expert=N_EXPERT):
    return rng.standard_normal((T, n_expert), dtype=np.float32)


def zipf_logits(rng, T, n_expert=N_EXPERT, k=TOP_K, s=1.1):
    """Logits whose top-k picks follow Zipf(s) expert popularity: each token
    draws k distinct experts with probability proportional to 1/rank^s over a
    seeded random ranking, and those get logits 8 + N(0,1) above the rest."""
    order = rng.permutation(n_expert)
    p = 1.0 / np.arange(1, n_expert + 1) ** s
    p /= p.sum()
    logits = rng.standard_normal((T, n_expert), dtype=np.float32)
    for t in range(T):
        picks = rng.choice(n_expert, size=k, replace=False, p=p)
        logits[t, order[picks]] += np.float32(8.0) + rng.standard_normal(k).astype(np.float32)
    return logits


def mixed_batch_tokens():
    """Config 5: 6 decode sequences of 1 token + prefill chunks of 3000, 1000."""
    return 6 + 3000 + 1000


def config_inputs(name, seed):
    """(x [T, D] f32, logits [T, E] f32, shg [T] f32 or None) for a named
    configuration: decode1, ragged64, prefill4096, mixed."""
    rng = np.random.default_rng(seed)
    if name == "decode1":
        T = 1
        return hidden(rng, T), normal_logits(rng, T), None
    if name == "ragged64":
        T = 64
        return hidden(rng, T), zipf_logits(rng, T), None
    if name == "prefill4096":
        T = 4096
        return hidden(rng, T), normal_logits(rng, T), None
    if name == "mixed":
        T = mixed_batch_tokens()
        return hidden(rng, T), normal_logits(rng, T), rng.standard_normal(T, dtype=np.float32)
    raise ValueError(name)
