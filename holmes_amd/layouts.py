"""Feature-major prefill layout (llama3fhe/layouts/feature_major.py:11-110): a ciphertext owns a
contiguous shard of tokens; inside it slot(dim, local_token) = dim * tokens_per_cipher + token.
The production contract is S = 128, D = 4096, slots = 32768: 8 tokens per ciphertext, 16
ciphertexts."""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def _pow2(value: int, name: str) -> None:
    if int(value) <= 0 or int(value) & (int(value) - 1):
        raise ValueError(f"{name} must be a positive power of two, got {value}.")


@dataclass(frozen=True)
class FeatureMajorPrefillLayout:
    seq_len: int = 128
    hidden_dim: int = 4096
    slots: int = 32768

    def __post_init__(self) -> None:
        _pow2(self.hidden_dim, "hidden_dim")
        if int(self.seq_len) <= 0:
            raise ValueError(f"seq_len must be positive, got {self.seq_len}.")
        if int(self.slots) % int(self.hidden_dim):
            raise ValueError("feature-major layout requires slots divisible by hidden_dim.")

    @property
    def tokens_per_cipher(self) -> int:
        return int(self.slots) // int(self.hidden_dim)

    @property
    def cipher_count(self) -> int:
        return -(-int(self.seq_len) // self.tokens_per_cipher)

    def slot(self, dim: int, local_token: int) -> int:
        if not 0 <= int(dim) < int(self.hidden_dim):
            raise IndexError(f"dim={dim} is outside [0, {self.hidden_dim}).")
        if not 0 <= int(local_token) < self.tokens_per_cipher:
            raise IndexError(f"local_token={local_token} is outside [0, {self.tokens_per_cipher}).")
        return int(dim) * self.tokens_per_cipher + int(local_token)

    def pack(self, rows: np.ndarray, *, dtype=np.float64) -> np.ndarray:
        """[seq_len][hidden_dim] -> [cipher_count][slots] (missing tokens are zero)."""

        rows = np.asarray(rows, dtype=dtype)
        if rows.shape != (int(self.seq_len), int(self.hidden_dim)):
            raise ValueError(f"feature-major rows must have shape {(self.seq_len, self.hidden_dim)}.")
        t = self.tokens_per_cipher
        padded = np.zeros((self.cipher_count * t, int(self.hidden_dim)), dtype=dtype)
        padded[: int(self.seq_len)] = rows
        # cipher c, slot d * t + j  <-  token c * t + j, feature d
        return padded.reshape(self.cipher_count, t, int(self.hidden_dim)).transpose(0, 2, 1).reshape(
            self.cipher_count, int(self.slots))

    def unpack(self, slots: np.ndarray) -> np.ndarray:
        """[cipher_count][slots] -> [seq_len][hidden_dim]."""

        slots = np.asarray(slots)
        t = self.tokens_per_cipher
        x = slots.reshape(self.cipher_count, int(self.hidden_dim), t).transpose(0, 2, 1)
        return x.reshape(self.cipher_count * t, int(self.hidden_dim))[: int(self.seq_len)]


__all__ = ["FeatureMajorPrefillLayout"]
