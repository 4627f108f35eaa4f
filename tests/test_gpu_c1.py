"""The C1 checkpoint-boundary codec on the GPU (stacr/protocols/checkpointing.py:176-587).

Kernel parity (through the C ABI) against the oracle on the kernels' own fp32 coefficients: the
observe pass's flags and max |.| exactly, the fp64 sums within 1e-9 and the energy within 1e-6
(the partial sums are combined in another order), the per-component scales, int8 codes and
dtype-cast coefficients bit for bit, and the reconstruction bit for bit (the same fp32 chain).
Codec behaviour: the reference's own record/refresh test (tests/test_checkpoint_boundary.py:155-167),
the dense fallbacks and their reasons, the first non-finite event, quantized records, counters and
statistics, and a GPT-2-medium boundary (8 x 1024 x 1024 bf16, rank 96) restored within fp32 / bf16
rounding of the fp64 reconstruction.
"""
import math
from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    return torch.device("cuda:0")


def announce(*parts):
    print("CASE", *parts, flush=True)


def _np(t):
    return t.detach().float().cpu().numpy()


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _basis(h, r, seed=1):
    g = torch.Generator().manual_seed(seed)
    return torch.linalg.qr(torch.randn(h, r, generator=g, dtype=torch.float64))[0].float()


def _boundary(rows, h, r, seed=2, noise=0.05):
    g = torch.Generator().manual_seed(seed)
    q = _basis(h, r, seed + 7)
    return torch.randn(rows, r, generator=g) @ q.t() * 3 + noise * torch.randn(rows, h, generator=g)


@pytest.mark.parametrize("rows,h,r,xdt,bdt,special", [
    (300, 64, 8, "f32", "f32", None), (1000, 256, 16, "bf16", "f32", "nan"), (77, 300, 5, "f16", "bf16", "inf"),
    (640, 1024, 96, "bf16", "f32", None), (129, 512, 64, "f32", "f16", "nan_inf"), (64, 32, 128, "f32", "f32", None),
])
def test_c1_kernels_match_oracle(dev, rows, h, r, xdt, bdt, special):
    from stacr_amd import kernels

    announce("c1 kernels", rows, h, r, xdt, bdt, special)
    x = _boundary(rows, h, min(r, h), seed=rows)
    if special in ("nan", "nan_inf"):
        x[3, 5] = float("nan")
    if special in ("inf", "nan_inf"):
        x[rows - 1, h - 1] = float("inf")
    xd = x.to(dev, DT[xdt])
    qd = _basis(h, r, 3).to(dev, DT[bdt])
    coeff = xd.float() @ qd.float()
    stats, scales = kernels.c1_observe(xd, coeff, qd)
    torch.cuda.synchronize()
    got = kernels.c1_parse_stats(stats)
    want = orc.c1_observe(_np(xd), _np(coeff), _np(qd))
    assert got["flags"] == want["flags"]
    for k in ("input_max_abs", "coeff_max_abs", "reconstruction_max_abs", "residual_max_abs", "basis_max_abs"):
        assert got[k] == np.float32(want[k]), k
    for k, tol in (("error", 1e-9), ("denom", 1e-9), ("energy", 1e-6)):
        a, b = got[k], want[k]
        assert a == b or (math.isnan(a) and math.isnan(b)) or math.isclose(a, b, rel_tol=tol), k
    s_want = orc.c1_scales(_np(coeff))
    assert np.array_equal(_bits(_np(scales)), _bits(s_want))
    codes = kernels.c1_store(coeff, scales, True, torch.int8)
    assert np.array_equal(codes.cpu().numpy(), orc.c1_store(_np(coeff), s_want, "f32"))
    stored = kernels.c1_store(coeff, None, False, DT[bdt])
    assert np.array_equal(_bits(_np(stored)), _bits(orc.c1_store(_np(coeff), None, bdt)))
    for c, s in ((codes, scales), (stored, None)):
        out = kernels.c1_restore(c, s, qd, DT[xdt])
        ref = orc.c1_restore(c.cpu().numpy() if s is not None else _np(c), None if s is None else _np(s), _np(qd), xdt)
        assert out.dtype == DT[xdt] and np.array_equal(_bits(_np(out)), _bits(ref))


def boundary_spec(**overrides):
    from stacr_amd.checkpoint_codec import STACRCheckpointSpec

    spec = STACRCheckpointSpec(site_id="block", module_type="GPT2Block", model_family="gpt2", hidden_size=32, rank=8,
                               residual_mode="none", residual_budget=0, basis_dtype=torch.float32,
                               quantize_coefficients=False, quantize_bits=8, quantize_residuals=False,
                               residual_quantize_bits=4, warmup_steps=1, refresh_trigger="off", refresh_period=1,
                               refresh_energy_threshold=0.15, target_arg_index=0, min_numel=1)
    return replace(spec, **overrides)


def test_record_reconstruction_survives_later_basis_refresh(dev):
    """Reference tests/test_checkpoint_boundary.py:155-167 on the GPU."""
    from stacr_amd.checkpoint_codec import CheckpointBoundaryCodec, _deserialize_packed_record, _serialize_packed_record

    announce("c1 record survives refresh")
    torch.manual_seed(16)
    codec = CheckpointBoundaryCodec(boundary_spec(refresh_trigger="period", refresh_period=2))
    codec.pack_tensor(torch.randn(2, 8, 32, device=dev), training=True)
    record = codec.pack_tensor(torch.randn(2, 8, 32, device=dev), training=True)
    assert not record.is_dense_fallback
    expected = codec.unpack_record(record).clone()
    codec.pack_tensor(torch.randn(2, 8, 32, device=dev), training=True)
    refreshed = codec.pack_tensor(torch.randn(2, 8, 32, device=dev), training=True)
    assert refreshed.is_dense_fallback
    meta, tensors = _serialize_packed_record(record)
    restored = _deserialize_packed_record(meta, tuple(tensors))
    torch.testing.assert_close(codec.unpack_record(restored), expected)
    st = codec.stats()
    assert st["fallback_reasons"] == {"warmup_dense": 1, "trigger_refresh_dense": 1}
    assert st["basis_refresh_count"] == 2 and st["basis_warmup_refresh_count"] == 1
    assert st["basis_trigger_refresh_count"] == 1 and st["step_count"] == 4 and st["pack_count"] == 4


@pytest.mark.parametrize("quantized,basis_dtype", [(False, torch.float32), (True, torch.float32),
                                                   (False, torch.bfloat16)])
def test_compressed_record_round_trip(dev, quantized, basis_dtype):
    from stacr_amd.checkpoint_codec import CheckpointBoundaryCodec

    announce("c1 round trip", quantized, basis_dtype)
    codec = CheckpointBoundaryCodec(boundary_spec(hidden_size=64, warmup_steps=0, quantize_coefficients=quantized,
                                                  basis_dtype=basis_dtype))
    x = _boundary(4 * 16, 64, 8, seed=11, noise=0.0).reshape(4, 16, 64).to(dev)
    rec = codec.pack_tensor(x, training=True)
    assert not rec.is_dense_fallback and rec.coeff.shape == (4, 16, 8)
    assert rec.coeff.dtype == (torch.int8 if quantized else basis_dtype)
    assert (rec.coeff_scale is not None) == quantized and rec.coeff_quantized == quantized
    if quantized:
        assert rec.coeff_scale.shape == (1, 1, 8) and rec.coeff_scale.dtype == torch.float32
    out = codec.unpack_record(rec)
    assert out.shape == x.shape and out.dtype == x.dtype
    # the record against the oracle: stored coefficients, then the fp32 chain
    want = orc.c1_restore(rec.coeff.reshape(-1, 8).cpu().numpy() if quantized else _np(rec.coeff.reshape(-1, 8)),
                          _np(rec.coeff_scale.reshape(-1)) if quantized else None, _np(rec.basis), "f32")
    assert np.array_equal(_bits(_np(out).reshape(-1, 64)), _bits(want))
    # a rank-8 boundary on its own SVD basis comes back within the coefficient rounding
    tol = 2e-2 if quantized or basis_dtype != torch.float32 else 1e-5
    assert torch.linalg.norm(out - x) / torch.linalg.norm(x) <= tol
    st = codec.stats()
    assert st["compressed_pack_count"] == 1 and st["basis_init_refresh_count"] == 1 and st["unpack_count"] == 1
    assert st["stored_bytes_total"] == rec.coeff.numel() * rec.coeff.element_size() + (32 if quantized else 0)
    assert st["raw_bytes_total"] == x.numel() * 4
    assert st["last_energy"] < (1e-6 if basis_dtype == torch.float32 else 1e-3)
    assert st["last_basis_max_abs"] is not None


def test_fallbacks_and_first_nonfinite(dev):
    from stacr_amd.checkpoint_codec import CheckpointBoundaryCodec

    announce("c1 fallbacks")
    x = _boundary(32, 32, 4, seed=5).reshape(2, 16, 32).to(dev)
    assert CheckpointBoundaryCodec(boundary_spec()).pack_tensor(x, training=False).is_dense_fallback
    unsupported = CheckpointBoundaryCodec(boundary_spec(residual_mode="topk"))
    assert unsupported.pack_tensor(x, training=True).is_dense_fallback
    assert unsupported.stats()["fallback_reasons"] == {"residual_mode_unsupported": 1}
    codec = CheckpointBoundaryCodec(boundary_spec(warmup_steps=0))
    bad = x.clone()
    bad[0, 3, 4] = float("nan")
    bad[1, 0, 0] = float("inf")
    rec = codec.pack_tensor(bad, training=True)
    assert rec.is_dense_fallback and rec.dense_tensor is bad
    st = codec.stats()
    assert st["fallback_reasons"] == {"input_nonfinite": 1}
    assert st["first_nonfinite_reason"] == "input_nonfinite" and st["first_nonfinite_stage"] == "input"
    assert st["first_nonfinite_step"] == 1
    assert st["first_nonfinite_input_max_abs"] == 3.4028234663852886e38  # a NaN and an inf: nan_to_num's max
    assert st["last_input_max_abs"] == 3.4028234663852886e38 and st["last_coeff_max_abs"] is None
    assert not st["basis_initialized"]  # the input check comes before the basis
    energy = CheckpointBoundaryCodec(boundary_spec(warmup_steps=0, refresh_trigger="residual_energy",
                                                   refresh_energy_threshold=1e-9, rank=2))
    first = energy.pack_tensor(x, training=True)  # init, then the energy is over the threshold
    assert first.is_dense_fallback and energy.stats()["fallback_reasons"] == {"trigger_refresh_dense": 1}
    assert energy.stats()["basis_init_refresh_count"] == 1 and energy.stats()["basis_trigger_refresh_count"] == 1


def test_gpt2_medium_boundary(dev):
    """A GPT-2-medium block input (batch 8, seq 1024, hidden 1024, bf16) at the default GPT-2 rank 96."""
    from stacr_amd.checkpoint_codec import CheckpointBoundaryCodec

    announce("c1 gpt2-medium boundary")
    x = _boundary(8192, 1024, 64, seed=3, noise=0.02).reshape(8, 1024, 1024).to(dev, torch.bfloat16)
    codec = CheckpointBoundaryCodec(boundary_spec(hidden_size=1024, rank=96, warmup_steps=0))
    rec = codec.pack_tensor(x, training=True)
    assert not rec.is_dense_fallback
    out = codec.unpack_record(rec)
    q64 = rec.basis.double()
    ref = (x.reshape(-1, 1024).double() @ q64) @ q64.t()
    assert torch.linalg.norm(out.reshape(-1, 1024).double() - ref) / torch.linalg.norm(ref) <= 4e-3
    st = codec.stats()
    xf, c = x.reshape(-1, 1024).float(), x.reshape(-1, 1024).float() @ codec.basis.float()
    want = orc.c1_observe(_np(xf), _np(c), _np(codec.basis))
    assert math.isclose(st["last_energy"], want["energy"], rel_tol=1e-5)
