"""The reference's FlexAttention descriptions of its variants (extra_bench.py:81-95),
restated as predicates and modifiers for the flex tests (16 heads)."""
import torch

H_REF = 16
TEMPS = 0.5 + torch.arange(H_REF, dtype=torch.float32) / H_REF   # extra_bench.py:83 (float32)
SLOPES = torch.arange(1, H_REF + 1, dtype=torch.float32)          # extra_bench.py:82


def causal(b, h, q, k):
    return k <= q


# (variant, score modifier, mask predicate)
FLEX_REF = [
    ("temp_perhead", lambda s, b, h, q, k: s * TEMPS[h], causal),
    ("bias_alibi", lambda s, b, h, q, k: s + SLOPES[h] * (k - q), causal),
    ("softcap_gemma2", lambda s, b, h, q, k: torch.tanh(s / 30.0) * 30.0, causal),
    ("bias_dilated", None, lambda b, h, q, k: (k <= q) & ((q - k) % 4 == 0)),
    ("bias_local", None, lambda b, h, q, k: (q - k).abs() < 256),
    ("bias_block_diagonal", None, lambda b, h, q, k: (q // 512 == k // 512) & (k <= q)),
    ("bias_prefix_lm", None, lambda b, h, q, k: (k <= q) | (k < 256)),
    ("bias_sliding_window", None, lambda b, h, q, k: (k <= q) & (q - k < 256)),
]
