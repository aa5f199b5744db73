"""Model configuration for the speculative-decoding engine.

`GPTConfig` mirrors the reference's frozen dataclass field for field
(flaxchat/config.py:16-27) and adds one optional field, `short_window`,
because the reference derives the short sliding window from
`sequence_len` (flaxchat/gpt.py:318-319) while the benchmark
configurations state it explicitly.
"""

from __future__ import annotations

from dataclasses import dataclass, field, replace
from typing import List, Optional, Tuple


@dataclass(frozen=True)
class GPTConfig:
    """Architecture of a flaxchat GPT (flaxchat/config.py:16-27).

    short_window: left window of "S" layers. None keeps the reference rule
    ceil(sequence_len / 4 / 128) * 128 (flaxchat/gpt.py:318-319).
    """
    sequence_len: int = 2048
    vocab_size: int = 32768
    n_layer: int = 12
    n_head: int = 6
    n_kv_head: int = 6
    n_embd: int = 768
    window_pattern: str = "SSSL"
    tie_embeddings: bool = False
    use_scan: bool = False
    short_window: Optional[int] = None

    @property
    def head_dim(self) -> int:
        return self.n_embd // self.n_head

    def with_(self, **kw) -> "GPTConfig":
        return replace(self, **kw)


def has_ve(layer_idx: int, n_layer: int) -> bool:
    """Value-embedding layers: alternate, last layer always included
    (flaxchat/gpt.py:77-79)."""
    return layer_idx % 2 == (n_layer - 1) % 2


def compute_window_sizes(config: GPTConfig) -> List[Tuple[int, int]]:
    """Per-layer (left, right) windows (flaxchat/gpt.py:313-327).

    The last layer is always full ("L") width. The decode mask is
    `pos - j <= left` (inclusive: left + 1 keys), applied when left > 0
    (flaxchat/engine.py:148-151).
    """
    pattern = config.window_pattern.upper()
    if not pattern or any(c not in "SL" for c in pattern):
        raise ValueError(f"Invalid window_pattern: {config.window_pattern!r}")
    long_window = config.sequence_len
    if config.short_window is None:
        short_window = -(-long_window // 4 // 128) * 128
    else:
        short_window = int(config.short_window)
    char_to_window = {"L": (long_window, 0), "S": (short_window, 0)}
    sizes = [char_to_window[pattern[i % len(pattern)]] for i in range(config.n_layer)]
    sizes[-1] = (long_window, 0)
    return sizes


def padded_vocab(config: GPTConfig, pad_to: int = 64) -> int:
    """Vocabulary padded to a multiple of 64 (flaxchat/gpt.py:217)."""
    return ((config.vocab_size + pad_to - 1) // pad_to) * pad_to
