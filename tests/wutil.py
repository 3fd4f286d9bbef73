"""Shared helpers of the weight-format tests: random ggml-format weight rows with finite fp16 scales."""
import numpy as np

import oracle as O

# byte offsets of the fp16 scale fields inside one 256-weight block
SCALE_OFFSETS = {O.W_Q4_K: [0, 2], O.W_Q2_K: [80, 82], O.W_Q6_K: [208], O.W_IQ4_XS: [0], O.W_IQ2_XXS: [0],
                 O.W_IQ2_XS: [0], O.W_IQ2_S: [0], O.W_IQ3_XXS: [0], O.W_IQ3_S: [0]}


def random_rows(fmt, N, K, seed, scale=0.01):
    """Random bytes, with every block's d / dmin field rewritten as a small normal fp16 value."""
    rng = np.random.default_rng(seed)
    rb = O.w_row_bytes(fmt, K)
    W = rng.integers(0, 256, (N, rb), dtype=np.uint8)
    blocks = W.reshape(N, K // 256, rb // (K // 256))
    for o in SCALE_OFFSETS[fmt]:
        vals = (rng.standard_normal(blocks.shape[:2]) * scale).astype(np.float16).view(np.uint16)
        blocks[:, :, o] = (vals & 255).astype(np.uint8)
        blocks[:, :, o + 1] = (vals >> 8).astype(np.uint8)
    return W
