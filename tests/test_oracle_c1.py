"""Oracle pins for the C1 checkpoint-boundary codec's device work
(stacr/protocols/checkpointing.py:374-400,411-545): the residual energy against closed forms and
against torch's CPU ops of the reference's sequence, the per-component scales and int8 codes
against torch's CPU ops of _quantize_coefficients (bit for bit), the max-abs convention against a
torch restatement of _safe_max_abs, and the reconstruction through lowrank (pinned elsewhere
against torch's mm)."""
import math

import numpy as np
import torch

from oracle import oracle as orc


def _torch_safe_max_abs(t: torch.Tensor) -> float:
    a = t.abs()
    m = a.amax()
    if torch.isfinite(m) or torch.isinf(m):
        return float(m)
    if torch.isnan(a).all():
        return float("nan")
    return float(torch.nan_to_num(a, nan=0.0).amax())


def _orthonormal(h, r, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.linalg.qr(torch.randn(h, r, generator=g, dtype=torch.float64))[0].float()


def test_c1_energy_closed_forms():
    q = torch.zeros(16, 4)
    q[torch.arange(4), torch.arange(4)] = 1.0  # unit basis vectors: exact products
    c = torch.tensor([[1.0, -2.0, 0.5, 3.0], [0.0, 0.0, 0.0, 0.0]])
    x = c @ q.t()
    x[1, 7] = 2.0  # the second row lies outside the span: all of it is residual
    s = orc.c1_observe(x.numpy(), c.numpy(), q.numpy())
    assert s["error"] == 4.0 and s["denom"] == float((x * x).sum())
    assert s["energy"] == np.float32(4.0) / np.float32(s["denom"])
    outside = orc.c1_observe(x[1:].numpy(), c[1:].numpy(), q.numpy())
    assert outside["energy"] == 1.0 and outside["residual_max_abs"] == 2.0
    inside = orc.c1_observe(x[:1].numpy(), c[:1].numpy(), q.numpy())
    assert inside["energy"] == 0.0 and inside["flags"] == 16 | 32 | 64 | 128 | 256  # no NaN anywhere


def test_c1_energy_against_torch_sequence():
    g = torch.Generator().manual_seed(5)
    q = _orthonormal(64, 8, 1)
    x = torch.randn(300, 8, generator=g) @ q.t() + 0.1 * torch.randn(300, 64, generator=g)
    coeff = x @ q  # the reference's flat_fp32 @ basis_fp32
    recon = coeff @ q.t()
    resid = x - recon
    ref = float(resid.pow(2).sum() / x.pow(2).sum().clamp_min(1e-12))
    s = orc.c1_observe(x.numpy(), coeff.numpy(), q.numpy())
    assert math.isclose(s["energy"], ref, rel_tol=1e-4)
    assert s["residual_max_abs"] == _torch_safe_max_abs(torch.from_numpy(x.numpy() - orc.lowrank(coeff.numpy(), q.numpy(), "f32")))
    assert s["input_max_abs"] == _torch_safe_max_abs(x) and s["basis_max_abs"] == _torch_safe_max_abs(q)


def test_c1_max_abs_convention_and_flags():
    q = _orthonormal(8, 2, 2)
    x = torch.ones(4, 8)
    x[0, 0], x[1, 1], x[2, 2] = float("nan"), float("inf"), -5.0
    c = torch.ones(4, 2)
    s = orc.c1_observe(x.numpy(), c.numpy(), q.numpy())
    # a NaN and an inf: the largest finite float (torch.nan_to_num clamps the inf), reported here as
    # the NaN flag with max inf
    assert s["flags"] & 1 and s["flags"] & 16 and s["input_max_abs"] == math.inf
    assert _torch_safe_max_abs(x) == 3.4028234663852886e38
    x[0, 0] = 1.0  # inf without a NaN: inf
    assert orc.c1_observe(x.numpy(), c.numpy(), q.numpy())["flags"] & 1 == 0 and _torch_safe_max_abs(x) == math.inf
    allnan = orc.c1_observe(np.full((2, 8), np.nan, np.float32), c[:2].numpy(), q.numpy())
    assert not allnan["flags"] & 16 and math.isnan(_torch_safe_max_abs(torch.full((2, 8), float("nan"))))


def _torch_quantize(coeff: torch.Tensor):
    """The reference's _quantize_coefficients on a (rows, rank) tensor (:374-393)."""
    max_abs = coeff.detach().abs().to(torch.float32).amax(dim=(0,), keepdim=True)
    safe = torch.where(torch.isfinite(max_abs) & (max_abs > 0), max_abs, torch.ones_like(max_abs))
    scale = safe / 127.0
    return torch.clamp(torch.round(coeff.to(torch.float32) / scale), -127, 127).to(torch.int8), scale.reshape(-1)


def test_c1_scales_and_codes_match_torch():
    g = torch.Generator().manual_seed(8)
    c = torch.randn(500, 12, generator=g) * torch.exp(torch.randn(1, 12, generator=g) * 3)
    c[:, 3] = 0.0           # an all-zero component: scale 1 / 127
    c[7, 5] = float("inf")  # an infinite one: scale 1 / 127, the inf codes 127
    c[9, 6] = float("nan")  # NaN propagates through amax: scale 1 / 127
    tq, ts = _torch_quantize(c)
    s = orc.c1_scales(c.numpy())
    assert np.array_equal(s, ts.numpy())
    codes = orc.c1_store(c.numpy(), s, "f32")
    finite = torch.isfinite(c).numpy()
    assert np.array_equal(codes[finite], tq.numpy()[finite]) and codes[7, 5] == 127 and codes[9, 6] == 0
    # the largest magnitude of a component with a positive finite max codes to +-127
    assert (np.abs(codes[:, [0, 1, 2, 4]]).max(axis=0) == 127).all()


def test_c1_restore_dequantizes_then_chains():
    q = _orthonormal(32, 4, 3).numpy()
    codes = np.array([[127, -3, 0, 5], [1, 2, -127, 0]], np.int8)
    s = np.array([0.5, 0.25, 2.0, 1.0], np.float32)
    out = orc.c1_restore(codes, s, q, "f32")
    want = orc.lowrank((codes.astype(np.float32) * s).astype(np.float32), q, "f32")
    assert np.array_equal(out, want)
    ref = (torch.from_numpy(codes).float() * torch.from_numpy(s)) @ torch.from_numpy(q).t()
    assert np.allclose(out, ref.numpy(), rtol=1e-6, atol=1e-6)
