"""Compact forms of a save's outputs, on the HIP codecs.

``IndexStream``: the residual's sorted flat indices as a bit-packed delta stream (blocks of 256
entries, one bit width per block), a denser form of the reference's delta codec
(stacr/index_compression.py:231-269) that decodes back to the same indices (``decode``, the
base-plus-cumulative-deltas rule of :327-342).  The drop-in layers keep saving flat int32
indices, as the reference's tests read them back from ``grad_fn.saved_tensors``; the stream is
for callers that store or move the residual.

``RowQuantizedCoefficients``: int8 coefficients with one fp32 scale per row (the C1 checkpoint
codec's safe-max rule, stacr/protocols/checkpointing.py:374-400, taken per row).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import kernels

_STATUS_REASONS = {1: "indices are not non-decreasing", 2: "a gap between indices is 2^32 or more",
                   4: "an index is negative"}


@dataclass
class IndexStream:
    nnz: int
    base: torch.Tensor      # int64[nb]: each block's first index
    word_off: torch.Tensor  # int32[nb + 1]: uint32 word offsets of the blocks; word_off[nb] = length
    words: torch.Tensor     # int32: the packed deltas (uint32 bit patterns), at least the length
    status: torch.Tensor    # int32[1]: 0, or the OR of the reasons the input could not be stored

    @classmethod
    def encode(cls, indices: torch.Tensor) -> "IndexStream":
        base, word_off, words, status = kernels.index_stream_encode(indices)
        return cls(int(indices.numel()), base, word_off, words, status)

    def decode(self, dtype: torch.dtype = torch.int32) -> torch.Tensor:
        return kernels.index_stream_decode(self.base, self.word_off, self.words, self.nnz, dtype)

    def length_words(self) -> int:
        """Words the stream uses (reads one value from the device)."""
        return int(self.word_off[-1].item()) & 0xFFFFFFFF

    def check(self) -> "IndexStream":
        """Raise ValueError when the encoded input could not be represented (reads the status)."""
        code = int(self.status.item())
        if code:
            reasons = [msg for bit, msg in _STATUS_REASONS.items() if code & bit]
            raise ValueError("index stream: " + "; ".join(reasons))
        return self

    def trim(self) -> "IndexStream":
        """The same stream with its word buffer cut to the used length (one device read)."""
        n = self.length_words()
        return IndexStream(self.nnz, self.base, self.word_off, self.words[:n].clone(), self.status)

    def nbytes(self) -> int:
        """Bytes of the trimmed stream: bases, offsets and words."""
        return self.base.numel() * 8 + self.word_off.numel() * 4 + self.length_words() * 4


@dataclass
class RowQuantizedCoefficients:
    codes: torch.Tensor   # int8 rows x rank
    scales: torch.Tensor  # float32[rows]
    dtype: torch.dtype    # the coefficients' dtype

    @classmethod
    def quantize(cls, coeff: torch.Tensor) -> "RowQuantizedCoefficients":
        codes, scales = kernels.quantize_rows_int8(coeff)
        return cls(codes, scales, coeff.dtype)

    def dequantize(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        return kernels.dequantize_rows_int8(self.codes, self.scales, dtype or self.dtype)

    def nbytes(self) -> int:
        return self.codes.numel() + self.scales.numel() * 4


__all__ = ["IndexStream", "RowQuantizedCoefficients"]
