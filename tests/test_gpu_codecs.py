"""The compact save outputs on the GPU: the bit-packed index stream (stacr_index_stream_*) and
row-quantized int8 coefficients (stacr_*_rows_int8), bit-exact against the oracle's formats.

Streams are checked word for word (bases, offsets, the used words, status) and decoded back to the
input, including the indices of a full-size cfg3 c_fc save (41,943 entries), int64 indices past
2^32, duplicates, the widest gap (2^32 - 1), block-boundary sizes and the three status flags.
"""
import numpy as np
import pytest
import torch

from gpu_cases import make_activation, make_basis
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    return torch.device("cuda:0")


def announce(*parts):
    print("CASE", *parts, flush=True)


def _u32(t):
    return t.cpu().numpy().view(np.uint32)


def check_stream(dev, idx_np, idx_dtype):
    from stacr_amd.codecs import IndexStream

    idx = torch.from_numpy(np.asarray(idx_np)).to(dev, idx_dtype)
    s = IndexStream.encode(idx)
    torch.cuda.synchronize()
    base, off, words, status = orc.index_stream_encode(np.asarray(idx_np, np.int64))
    assert int(s.status.item()) == status
    assert np.array_equal(s.base.cpu().numpy(), base)
    assert np.array_equal(_u32(s.word_off), off)
    n = s.length_words()
    assert n == int(off[-1]) and np.array_equal(_u32(s.words)[:n], words)
    if status == 0:
        for out in (torch.int64, idx_dtype):
            back = s.decode(out)
            assert back.dtype == out and np.array_equal(back.cpu().numpy().astype(np.int64), np.asarray(idx_np, np.int64))
        t = s.trim()
        assert t.words.numel() == n and np.array_equal(t.decode(torch.int64).cpu().numpy(), np.asarray(idx_np, np.int64))
        assert s.nbytes() == base.size * 8 + off.size * 4 + n * 4
    return s


@pytest.mark.parametrize("n,span,dtype", [(0, 1, torch.int32), (1, 100, torch.int32), (255, 10**4, torch.int32),
                                          (256, 10**6, torch.int32), (257, 64, torch.int32),
                                          (20000, 8192 * 4096, torch.int32), (3000, 2**40, torch.int64),
                                          (70000, 2**33, torch.int64)])
def test_index_stream_matches_oracle(dev, n, span, dtype):
    announce("index stream", n, span, dtype)
    rng = np.random.default_rng(n)
    idx = np.sort(rng.integers(0, span, n, dtype=np.int64))
    check_stream(dev, idx, dtype)


def test_index_stream_of_a_full_save(dev):
    """The residual indices of the north-star layer's save (cfg3 c_fc, global top-k 0.005)."""
    from stacr_amd import kernels

    announce("index stream of cfg3 c_fc save")
    x = make_activation(8192, 1024, lognormal=True).to(dev, torch.bfloat16)
    q = make_basis(1024, 8).to(dev, torch.bfloat16)
    _, idx, _, _ = kernels.save(x, q, mode="global_topk", budget=0.005, chunk_rows=512, bits=8)
    assert idx.numel() == 41943
    s = check_stream(dev, idx.cpu().numpy().astype(np.int64), torch.int32)
    assert s.nbytes() < idx.numel() * 4 // 2  # gaps of about 200 need 8-9 bits, not 32


def test_index_stream_edges_and_status(dev):
    announce("index stream edges")
    check_stream(dev, np.array([3, 3, 3, 4, 4, 9]), torch.int32)          # duplicates
    check_stream(dev, np.array([0, 2**32 - 1], np.int64), torch.int64)    # the widest gap
    check_stream(dev, np.arange(600) * 8 + 5, torch.int32)                # one width everywhere
    check_stream(dev, np.array([5, 4, 7]), torch.int32)                   # status 1
    check_stream(dev, np.array([0, 2**32], np.int64), torch.int64)        # status 2
    check_stream(dev, np.array([-3, 1]), torch.int32)                     # status 4
    from stacr_amd.codecs import IndexStream

    with pytest.raises(ValueError, match="non-decreasing"):
        IndexStream.encode(torch.tensor([5, 4], device=dev)).check()


@pytest.mark.parametrize("dtype,rows,rank", [(torch.bfloat16, 8192, 8), (torch.float16, 777, 16),
                                             (torch.float32, 300, 5), (torch.bfloat16, 64, 1),
                                             (torch.float32, 50, 32)])
def test_rows_int8_matches_oracle(dev, dtype, rows, rank):
    from stacr_amd.codecs import RowQuantizedCoefficients

    announce("rows int8", dtype, rows, rank)
    g = torch.Generator().manual_seed(rows + rank)
    c = (torch.randn(rows, rank, generator=g) * torch.exp(2 * torch.randn(rows, 1, generator=g))).to(dtype)
    c[0] = 0.0
    c[1, 0] = float("inf")
    c[2, rank - 1] = float("nan")
    c[3] = torch.linspace(-3.5, 3.5, rank).to(dtype)
    rq = RowQuantizedCoefficients.quantize(c.to(dev))
    torch.cuda.synchronize()
    oq, os_ = orc.quantize_rows_int8(c.float().numpy())
    assert np.array_equal(rq.codes.cpu().numpy(), oq)
    assert np.array_equal(rq.scales.cpu().numpy().view(np.uint32), os_.view(np.uint32))
    for out in (torch.float32, torch.bfloat16, torch.float16):
        back = rq.dequantize(out)
        want = orc.dequantize_rows_int8(oq, os_, {torch.float32: "f32", torch.bfloat16: "bf16",
                                                  torch.float16: "f16"}[out])
        assert back.dtype == out
        assert np.array_equal(back.float().cpu().numpy().view(np.uint32), want.astype(np.float32).view(np.uint32))
    assert rq.nbytes() == rows * rank + rows * 4
