"""Oracle pins for the compact save outputs: the bit-packed index stream and row-quantized int8
coefficients (the library's own formats; the reference holds the byte-wide delta codec,
stacr/index_compression.py:231-269,327-342, and the C1 codec's per-component quantizer,
stacr/protocols/checkpointing.py:374-400).

Pins: a known answer worked out by hand from the format (the reference's own DeltaEncodedIndices
example, stacr/index_compression.py:625-628), widths and sizes in closed form, round trips, decode
against the reference delta codec's oracle, status flags; the row quantizer against torch's CPU
ops of the C1 rule taken per row, and its closed-form bounds.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc


def test_index_stream_known_answer():
    # deltas 0, 2, 3, 3, 4 -> width 3; bits 0 | 2 << 3 | 3 << 6 | 3 << 9 | 4 << 12 = 18128; 8 * 3 words
    base, off, words, status = orc.index_stream_encode(np.array([10, 12, 15, 18, 22]))
    assert status == 0 and base.tolist() == [10] and off.tolist() == [0, 24]
    assert words.tolist() == [18128] + [0] * 23
    assert orc.index_stream_decode(base, off, words, 5).tolist() == [10, 12, 15, 18, 22]


def test_index_stream_widths_and_sizes():
    idx = np.arange(600, dtype=np.int64) * 8 + 5  # every gap 8 -> width 4, blocks of 256, 256, 88
    base, off, words, status = orc.index_stream_encode(idx)
    assert status == 0 and base.tolist() == [5, 2053, 4101] and off.tolist() == [0, 32, 64, 96]
    # slot j of a width-4 block: nibble j; slot 0 is 0, the rest 8
    assert words[0] == 0x88888880 and words[1] == 0x88888888 and words[32] == 0x88888880
    one = orc.index_stream_encode(np.array([7]))
    assert one[1].tolist() == [0, 0] and one[2].size == 0  # a single entry: width 0, no words
    dup = orc.index_stream_encode(np.array([3, 3, 3, 4]))
    assert dup[1].tolist() == [0, 8] and dup[2][0] == 1 << 3  # deltas 0 0 0 1 -> width 1
    wide = orc.index_stream_encode(np.array([0, 2**32 - 1], np.int64))
    assert wide[3] == 0 and wide[1].tolist() == [0, 256] and wide[2][1] == 0xFFFFFFFF
    empty = orc.index_stream_encode(np.zeros(0, np.int64))
    assert empty[0].size == 0 and empty[1].tolist() == [0] and empty[2].size == 0


@pytest.mark.parametrize("seed,n,span", [(0, 1, 10), (1, 255, 1000), (2, 256, 10**6), (3, 257, 50), (4, 3000, 2**40),
                                         (5, 5000, 5000)])
def test_index_stream_round_trip_matches_delta_codec(seed, n, span):
    rng = np.random.default_rng(seed)
    idx = np.sort(rng.integers(0, span, n, dtype=np.int64))  # duplicates allowed when span is small
    base, off, words, status = orc.index_stream_encode(idx)
    gaps = np.diff(idx)
    assert status == (2 if gaps.size and gaps.max() >= 2**32 else 0)
    if status == 0:
        assert np.array_equal(orc.index_stream_decode(base, off, words, n), idx)
        dbase, deltas = orc.delta_encode(idx, 1, int(idx.max()) + 1)
        assert np.array_equal(orc.delta_decode(dbase.astype(np.int64), deltas, n), idx)
        # size: 8 words per bit of each block's largest gap
        widths = [int(np.diff(idx[b:b + 256]).max(initial=0)).bit_length() for b in range(0, n, 256)]
        assert int(off[-1]) == 8 * sum(widths) == words.size


def test_index_stream_status_flags():
    assert orc.index_stream_encode(np.array([5, 4]))[3] == 1
    assert orc.index_stream_encode(np.array([0, 2**32], np.int64))[3] == 2
    assert orc.index_stream_encode(np.array([-1, 3]))[3] == 4


def _torch_rows_int8(c: torch.Tensor):
    """The C1 codec's quantizer (stacr/protocols/checkpointing.py:383-393) with the max per row."""
    max_abs = c.detach().abs().to(torch.float32).amax(dim=1, keepdim=True)
    safe = torch.where(torch.isfinite(max_abs) & (max_abs > 0), max_abs, torch.ones_like(max_abs))
    scale = safe / 127.0
    q = torch.clamp(torch.round(c.to(torch.float32) / scale), -127, 127).to(torch.int8)
    return q, scale.reshape(-1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_rows_int8_matches_torch_rule(dtype):
    g = torch.Generator().manual_seed(3)
    c = (torch.randn(300, 8, generator=g) * torch.exp(torch.randn(300, 1, generator=g))).to(dtype)
    c[5] = 0.0
    c[7, 3] = float("inf")
    c[9, :] = torch.tensor([0.5, -0.5, 1.5, -1.5, 2.5, 127.0, -127.0, 0.0]).to(dtype)  # ties at .5
    q, s = orc.quantize_rows_int8(c.float().numpy())
    tq, ts = _torch_rows_int8(c)
    assert np.array_equal(q, tq.numpy()) and np.array_equal(s, ts.numpy())
    assert s[5] == np.float32(1.0) / np.float32(127.0) and not q[5].any()
    assert q[7, 3] == 127  # inf / (1 / 127) clamps
    assert q[9].tolist() == [0, 0, 2, -2, 2, 127, -127, 0]  # scale 1: round half to even


def test_rows_int8_closed_form_bounds():
    rng = np.random.default_rng(9)
    c = (rng.standard_normal((500, 16)) * 10 ** rng.uniform(-3, 3, (500, 1))).astype(np.float32)
    q, s = orc.quantize_rows_int8(c)
    # the row's largest magnitude codes to +-127, every entry within half a step of its code
    assert np.array_equal(np.abs(q).max(axis=1), np.full(500, 127))
    err = np.abs(c - q.astype(np.float32) * s[:, None])
    assert (err <= 0.5 * s[:, None] * (1 + 1e-5)).all()
    # NaN in a row: the scale falls back to 1 / 127 and the NaN is coded 0
    c[0, 2] = np.nan
    q2, s2 = orc.quantize_rows_int8(c)
    assert s2[0] == np.float32(1.0) / np.float32(127.0) and q2[0, 2] == 0
    back = orc.dequantize_rows_int8(q, s, "bf16")
    assert np.array_equal(back, orc.round_to(q.astype(np.float32) * s[:, None], "bf16"))
