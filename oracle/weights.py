"""Counter-based random-init weights for the Qwen3 decode path (numpy, integer-only).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The benchmark configs ask for "BF16 weights ~N(0, 0.02) from seed 0". To make
"the same weights" mean the same BITS on every machine and library version,
each element is a pure function of ``(seed, tensor id, logical element index)``:

    key = seed << 52 | tensor_id << 32 | index          (index < 2**32)
    z   = splitmix64(key)                                (the published
          SplitMix64 output function: Steele, Lea, Flood, OOPSLA 2014)
    s   = sum of the four 16-bit fields of z  -  131070  (Irwin-Hall, n = 4)
    w   = bf16_rne( f32(s) * f32(std / sigma) ),   sigma = sqrt((65536**2 - 1) / 3)

``s`` has mean 0 and standard deviation ``sigma``, so ``w`` has standard
deviation ``std`` and an approximately normal (Irwin-Hall, bounded at 3.46
sigma) shape. Every step is exact integer arithmetic or one IEEE fp32 multiply
followed by round-to-nearest-even, so a GPU kernel doing the same steps gives
identical bits. RMSNorm gains are 1.0, as ``Qwen3RMSNorm`` initialises them
(``modeling_qwen3.py:56``).

Tensor ids: the embedding (tied with the LM head) is 0; the projections of
layer ``l`` are ``1 + 16 * l + j`` with ``j`` = 0 q_proj, 1 k_proj, 2 v_proj,
3 o_proj, 4 gate_proj, 5 up_proj, 6 down_proj. Logical indices are row-major
over the HF ``[out_features, in_features]`` weight shape.
"""

from __future__ import annotations

import math

import numpy as np

MASK64 = np.uint64(0xFFFFFFFFFFFFFFFF)
PROJ_IDS = {"q_proj": 0, "k_proj": 1, "v_proj": 2, "o_proj": 3, "gate_proj": 4, "up_proj": 5, "down_proj": 6}


def scale_f32(std: float) -> np.float32:
    """fp32 multiplier turning the centred Irwin-Hall sum into a ``std`` deviate."""
    sigma = math.sqrt((65536.0 * 65536.0 - 1.0) / 3.0)
    return np.float32(std / sigma)


def tensor_id(layer: int | None, name: str) -> int:
    if name == "embed":
        return 0
    return 1 + 16 * int(layer) + PROJ_IDS[name]


def splitmix64(key: np.ndarray) -> np.ndarray:
    """SplitMix64 output function on uint64 arrays (wrapping arithmetic)."""
    with np.errstate(over="ignore"):
        z = key + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def bf16_rne_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit pattern, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    return ((u + np.uint32(0x7FFF) + lsb) >> np.uint32(16)).astype(np.uint16)


def gen_bits(seed: int, tid: int, start: int, count: int, std: float = 0.02) -> np.ndarray:
    """bf16 bit patterns of elements ``[start, start + count)`` of tensor ``tid``."""
    idx = np.arange(start, start + count, dtype=np.uint64)
    key = (np.uint64(seed) << np.uint64(52)) | (np.uint64(tid) << np.uint64(32)) | idx
    z = splitmix64(key)
    m16 = np.uint64(0xFFFF)
    s = ((z & m16) + ((z >> np.uint64(16)) & m16) + ((z >> np.uint64(32)) & m16) + (z >> np.uint64(48)))
    s = s.astype(np.int64) - 131070
    v = s.astype(np.float32) * scale_f32(std)
    return bf16_rne_bits(v)


def gen_tensor_bits(seed: int, tid: int, shape, std: float = 0.02, chunk: int = 1 << 24) -> np.ndarray:
    """Whole tensor as bf16 bits (uint16), generated in chunks to bound memory."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.uint16)
    for s0 in range(0, n, chunk):
        c = min(chunk, n - s0)
        out[s0:s0 + c] = gen_bits(seed, tid, s0, c, std)
    return out.reshape(shape)


def bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def model_shapes(cfg: dict) -> dict:
    """HF weight shapes ``name -> [out, in]`` for one decoder layer."""
    H, I, D = cfg["hidden_size"], cfg["intermediate_size"], cfg["head_dim"]
    Nq, Nkv = cfg["num_attention_heads"], cfg["num_key_value_heads"]
    return {
        "q_proj": (Nq * D, H), "k_proj": (Nkv * D, H), "v_proj": (Nkv * D, H),
        "o_proj": (H, Nq * D), "gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I),
    }
