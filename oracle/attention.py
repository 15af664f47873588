"""Non-causal softmax attention over packed qkv rows, in float64.

qkv fp16 [S*L, 3C] (q pre-rotated and pre-scaled by softmax_scale * log2(e), k rotated; heads of 64 columns) ->
out fp16 [S*L, C]: per sequence and head, out = sum_j 2^(s_ij - max_j s_ij) v_j / sum_j 2^(s_ij - max_j s_ij)
with s_ij = q_i . k_j. Reference: attention_kernel, foidfinder/backends/cuda/csrc/attention.cuh:19-157 (its fp16
block accumulation is a precision choice of that kernel, not part of the op's definition).
"""

from __future__ import annotations

import numpy as np

D = 64


def attention(qkv: np.ndarray, seq_len: int, *, out_dtype=np.float16) -> np.ndarray:
    T, W = qkv.shape
    assert W % 3 == 0 and (W // 3) % D == 0 and T % seq_len == 0
    C = W // 3
    H = C // D
    S = T // seq_len
    out = np.empty((S, seq_len, H, D), out_dtype)
    for i in range(S):  # one sequence at a time keeps the [H, L, L] scores small
        x = qkv[i * seq_len : (i + 1) * seq_len].astype(np.float64).reshape(seq_len, 3, H, D)
        q = x[:, 0].transpose(1, 0, 2)  # [H, L, D]
        k = x[:, 1].transpose(1, 0, 2)
        v = x[:, 2].transpose(1, 0, 2)
        s = q @ k.transpose(0, 2, 1)
        s = s - s.max(axis=-1, keepdims=True)
        p = np.exp2(s)
        o = (p @ v) / p.sum(axis=-1, keepdims=True)
        out[i] = o.transpose(1, 0, 2).astype(out_dtype)
    return out.reshape(T, C)
