"""C1 checkpoint-boundary codec (interface of stacr/protocols/checkpointing.py:102-590).

A ``CheckpointBoundaryCodec`` stands at one activation-checkpoint boundary (a decoder block's
input).  ``pack_tensor`` stores the boundary as fp32 coefficients C = X Q on a persistent per-site
basis Q (optionally int8 with one scale per basis component), or keeps it dense when the protocol
says so: during warm-up, on non-finite values, when a refresh is due, or for residual modes it does
not support.  ``unpack_record`` rebuilds C Q^T in the boundary's dtype.

Device work: C is a library GEMM (the reference's ``flat_fp32 @ basis_fp32``); one HIP pass
(``stacr_c1_observe``) then reads X once and returns every quantity the protocol inspects: the
residual energy, the non-finite flags and the max |.| of X, C, the reconstruction, the residual and
the basis, and the per-component quantization scales.  One device read per pack replaces the
reference's separate reductions and ``.item()`` calls.  The records' coefficients come from
``stacr_c1_store`` and the reconstruction from ``stacr_c1_restore``.  The basis itself comes from an
SVD of the boundary (torch library calls, as in the reference).

Only the per-site codec is here; the site registry and the checkpoint autograd wiring around it are
the protocol library's and stay out of scope.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Dict, Optional, Tuple

import torch
from torch import nn

from . import kernels


@dataclass(frozen=True)
class STACRCheckpointSpec:
    """Per-site settings (stacr/protocols/checkpointing.py:124-141)."""

    site_id: str
    module_type: str
    model_family: str
    hidden_size: int
    rank: int
    residual_mode: str
    residual_budget: float
    basis_dtype: torch.dtype
    quantize_coefficients: bool
    quantize_bits: int
    quantize_residuals: bool
    residual_quantize_bits: int
    warmup_steps: int
    refresh_trigger: str
    refresh_period: int
    refresh_energy_threshold: float
    target_arg_index: int
    min_numel: int


@dataclass
class CompressedBoundaryRecord:
    """A packed boundary (:144-155): dense, or coefficients (+ scales) and the basis they used."""

    site_id: str
    original_shape: Tuple[int, ...]
    original_dtype: torch.dtype
    device: torch.device
    is_dense_fallback: bool
    dense_tensor: Optional[torch.Tensor] = None
    coeff: Optional[torch.Tensor] = None
    coeff_scale: Optional[torch.Tensor] = None
    coeff_quantized: bool = False
    basis: Optional[torch.Tensor] = None


def _dtype_name(dtype: torch.dtype) -> str:
    return {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}.get(dtype, str(dtype))


_FLT_MAX = 3.4028234663852886e38


class _Observation:
    """The observe pass's record.  Per tensor it holds the largest |v| that is not NaN and whether
    the tensor holds a NaN / a value that is not NaN; from these come the finite checks and the
    reference's max-abs convention (``_safe_max_abs``, :80-99: NaN when every value is NaN, the
    largest finite float when a NaN and an inf are both present, since ``torch.nan_to_num`` clamps
    the inf, else the max)."""

    _KEYS = {"input": "input", "coeff": "coeff", "reconstruction": "recon", "residual": "residual",
             "basis": "basis"}

    def __init__(self, raw: Dict[str, Any], scales: torch.Tensor, coeff: torch.Tensor):
        self.raw, self.scales, self.coeff = raw, scales, coeff
        self.flags = int(raw["flags"])

    def _flag(self, name: str) -> bool:
        return bool(self.flags & kernels.C1_FLAGS[name])

    def nonfinite(self, what: str) -> bool:
        return self._flag(f"{self._KEYS[what]}_nan") or math.isinf(float(self.raw[f"{what}_max_abs"]))

    def max_abs(self, what: str) -> float:
        key = self._KEYS[what]
        value = float(self.raw[f"{what}_max_abs"])
        if not self._flag(f"{key}_valid"):
            return float("nan")
        if self._flag(f"{key}_nan") and math.isinf(value):
            return _FLT_MAX
        return value

    @property
    def energy(self) -> float:
        return float(self.raw["energy"])


class CheckpointBoundaryCodec(nn.Module):
    """Per-site persistent boundary codec (:176-587): buffers, counters and statistics keep the
    reference's names, so state dicts and ``stats()`` read the same."""

    _COUNTERS = ("_step_counter", "_basis_refresh_count", "_basis_init_refresh_count",
                 "_basis_warmup_refresh_count", "_basis_trigger_refresh_count", "_pack_count", "_unpack_count",
                 "_fallback_count", "_compressed_pack_count", "_duplicate_pack_count", "_raw_bytes_total",
                 "_stored_bytes_total")

    def __init__(self, spec: STACRCheckpointSpec):
        super().__init__()
        self.spec = spec
        self.register_buffer("basis", torch.zeros(spec.hidden_size, spec.rank, dtype=spec.basis_dtype))
        self.register_buffer("_basis_initialized", torch.tensor(False, dtype=torch.bool))
        for name in self._COUNTERS:
            self.register_buffer(name, torch.tensor(0, dtype=torch.int64))
        self.register_buffer("_energy_ewma", torch.tensor(0.0, dtype=torch.float32))
        self.register_buffer("_last_energy", torch.tensor(0.0, dtype=torch.float32))
        self._fallback_reasons: Dict[str, int] = {}
        self._first_nonfinite_event: Optional[Dict[str, Any]] = None
        self._last: Dict[str, Optional[float]] = {k: None for k in ("input", "coeff", "reconstruction", "residual",
                                                                       "basis")}

    # ---------------------------------------------------------------- counters
    def _bump(self, name: str, by: int = 1) -> None:
        getattr(self, name).add_(int(by))

    def _count(self, name: str) -> int:
        return int(getattr(self, name).item())

    @property
    def pack_count(self) -> int:
        return self._count("_pack_count")

    @property
    def unpack_count(self) -> int:
        return self._count("_unpack_count")

    @property
    def basis_refresh_count(self) -> int:
        return self._count("_basis_refresh_count")

    @property
    def step_count(self) -> int:
        return self._count("_step_counter")

    @property
    def basis_initialized(self) -> bool:
        return bool(self._basis_initialized.item())

    def _ensure_device(self, device: torch.device) -> None:
        if self.basis.device != device:
            self.to(device=device)

    # ---------------------------------------------------------------- records
    def _store_accounting(self, raw_bytes: int, stored_bytes: int, compressed: bool) -> None:
        self._bump("_raw_bytes_total", raw_bytes)
        self._bump("_stored_bytes_total", stored_bytes)
        if compressed:
            self._bump("_compressed_pack_count")

    def _dense_record(self, tensor: torch.Tensor) -> CompressedBoundaryRecord:
        return CompressedBoundaryRecord(self.spec.site_id, tuple(tensor.shape), tensor.dtype, tensor.device, True,
                                        dense_tensor=tensor)

    def _fallback(self, tensor: torch.Tensor, reason: str) -> CompressedBoundaryRecord:
        self._bump("_fallback_count")
        self._fallback_reasons[reason] = self._fallback_reasons.get(reason, 0) + 1
        nbytes = tensor.numel() * tensor.element_size()
        self._store_accounting(nbytes, nbytes, compressed=False)
        return self._dense_record(tensor)

    def note_duplicate_pack(self, tensor: torch.Tensor) -> None:
        self._bump("_duplicate_pack_count")
        self._bump("_fallback_count")
        self._fallback_reasons["duplicate_target_save"] = self._fallback_reasons.get("duplicate_target_save", 0) + 1
        nbytes = tensor.numel() * tensor.element_size()
        self._store_accounting(nbytes, nbytes, compressed=False)

    def _note(self, obs: Optional[_Observation], stages: Tuple[str, ...]) -> None:
        """The last pack's max |.| for the named stages; the others are cleared (as the reference
        records only what it has computed at each return point)."""
        for key in self._last:
            self._last[key] = obs.max_abs(key) if obs is not None and key in stages else None

    def _first_nonfinite(self, obs: _Observation, reason: str, stage: str, stages: Tuple[str, ...]) -> None:
        if self._first_nonfinite_event is not None:
            return
        event = {"step": self.step_count + 1, "reason": reason, "stage": stage}
        for key in ("input", "coeff", "reconstruction", "residual", "basis"):
            event[f"{key}_max_abs"] = obs.max_abs(key) if key in stages else None
        self._first_nonfinite_event = event

    # ---------------------------------------------------------------- basis
    def _compute_basis(self, flat: torch.Tensor) -> torch.Tensor:
        """The top right-singular vectors of the boundary (QR of X^T when the SVD fails), completed
        to the spec's rank with an orthonormal complement when X has fewer directions (:300-341)."""
        hidden = flat.shape[-1]
        keep = min(self.spec.rank, flat.shape[0], hidden)
        out = torch.zeros(hidden, self.spec.rank, device=flat.device, dtype=torch.float32)
        if keep <= 0:
            return out.to(self.spec.basis_dtype)
        work = flat.detach().to(torch.float32)
        try:
            top = torch.linalg.svd(work, full_matrices=False)[2][:keep].transpose(0, 1)
        except RuntimeError:
            top = torch.linalg.qr(work.transpose(0, 1), mode="reduced")[0][:, :keep]
        out[:, :keep] = top
        extra = min(self.spec.rank - keep, hidden - keep)
        if extra > 0:
            eye = torch.eye(hidden, device=flat.device, dtype=torch.float32)
            rest = eye - top @ (top.transpose(0, 1) @ eye)
            out[:, keep:keep + extra] = torch.linalg.qr(rest, mode="reduced")[0][:, :extra]
        return out.to(self.spec.basis_dtype)

    def _refresh(self, flat: torch.Tensor, reason: str) -> None:
        # a new tensor: records packed earlier keep the basis they were packed with
        self.basis = self._compute_basis(flat).detach()
        self._basis_initialized.fill_(True)
        self._bump("_basis_refresh_count")
        self._bump({"warmup": "_basis_warmup_refresh_count",
                    "trigger": "_basis_trigger_refresh_count"}.get(reason, "_basis_init_refresh_count"))

    def _should_refresh(self, energy: float) -> bool:
        trigger = self.spec.refresh_trigger
        after = max(self.step_count - self.spec.warmup_steps, 0)
        periodic = after > 0 and after % max(self.spec.refresh_period, 1) == 0
        over = energy > self.spec.refresh_energy_threshold
        return {"period": periodic, "residual_energy": over, "hybrid": periodic or over}.get(trigger, False)

    # ---------------------------------------------------------------- pack / unpack
    def _observe(self, flat: torch.Tensor) -> _Observation:
        basis32 = self.basis.to(torch.float32)
        coeff = flat.to(torch.float32) @ basis32  # the reference's fp32 projection (library GEMM)
        stats, scales = kernels.c1_observe(flat, coeff, self.basis)
        return _Observation(kernels.c1_parse_stats(stats), scales, coeff)

    def pack_tensor(self, tensor: torch.Tensor, *, training: bool) -> CompressedBoundaryRecord:
        if not training:
            return self._dense_record(tensor)
        self._bump("_pack_count")
        self._ensure_device(tensor.device)
        try:
            return self._pack(tensor)
        finally:
            self._bump("_step_counter")

    def _pack(self, tensor: torch.Tensor) -> CompressedBoundaryRecord:
        spec = self.spec
        flat = tensor.reshape(-1, tensor.shape[-1])
        obs = self._observe(flat)
        self._note(obs, ("input",))
        if spec.residual_mode != "none":
            return self._fallback(tensor, "residual_mode_unsupported")
        if obs.nonfinite("input"):
            self._first_nonfinite(obs, "input_nonfinite", "input", ("input",))
            return self._fallback(tensor, "input_nonfinite")
        if self.step_count < spec.warmup_steps:
            self._refresh(flat, "warmup")
            self._note(self._observe(flat), ("input", "basis"))
            return self._fallback(tensor, "warmup_dense")
        if not self.basis_initialized:
            self._refresh(flat, "init")
            obs = self._observe(flat)
        if obs.nonfinite("basis"):
            self._note(obs, ("input", "basis"))
            self._first_nonfinite(obs, "basis_nonfinite", "basis", ("basis",))
            return self._fallback(tensor, "basis_nonfinite")
        if obs.nonfinite("coeff"):
            self._note(obs, ("input", "coeff", "basis"))
            self._first_nonfinite(obs, "projection_nonfinite", "coefficients", ("input", "coeff"))
            return self._fallback(tensor, "projection_nonfinite")
        if spec.quantize_coefficients and spec.quantize_bits != 8:
            raise ValueError("C1 checkpoint coefficient quantization supports only 8-bit coefficients; "
                             f"got {spec.quantize_bits}.")
        if obs.nonfinite("reconstruction"):
            self._note(obs, ("input", "coeff", "reconstruction", "basis"))
            self._first_nonfinite(obs, "reconstruction_nonfinite", "reconstruction",
                                  ("input", "coeff", "reconstruction"))
            return self._fallback(tensor, "reconstruction_nonfinite")
        self._note(obs, ("input", "coeff", "reconstruction", "residual", "basis"))
        energy = obs.energy
        if not math.isfinite(energy):
            self._first_nonfinite(obs, "energy_nonfinite", "reconstruction", ("input", "coeff", "reconstruction"))
            return self._fallback(tensor, "energy_nonfinite")
        self._last_energy.fill_(energy)
        self._energy_ewma.mul_(0.9).add_(0.1 * energy)
        if self._should_refresh(energy):
            self._refresh(flat, "trigger")
            return self._fallback(tensor, "trigger_refresh_dense")
        lead = tuple(tensor.shape[:-1])
        if spec.quantize_coefficients:
            coeff = kernels.c1_store(obs.coeff, obs.scales, True, torch.int8).reshape(*lead, spec.rank)
            scale = obs.scales.reshape(*([1] * len(lead)), spec.rank)
        else:
            coeff = kernels.c1_store(obs.coeff, None, False, self.basis.dtype).reshape(*lead, spec.rank)
            scale = None
        stored = coeff.numel() * coeff.element_size() + (scale.numel() * scale.element_size() if scale is not None else 0)
        self._store_accounting(tensor.numel() * tensor.element_size(), stored, compressed=True)
        return CompressedBoundaryRecord(spec.site_id, tuple(tensor.shape), tensor.dtype, tensor.device, False,
                                        coeff=coeff, coeff_scale=scale, coeff_quantized=scale is not None,
                                        basis=self.basis)

    def unpack_record(self, packed: CompressedBoundaryRecord) -> torch.Tensor:
        self._bump("_unpack_count")
        self._ensure_device(packed.device)
        if packed.is_dense_fallback:
            assert packed.dense_tensor is not None
            return packed.dense_tensor
        if packed.basis is None:
            raise ValueError("Compressed checkpoint record is missing its saved basis")
        assert packed.coeff is not None
        coeff = packed.coeff.reshape(-1, self.spec.rank)
        scale = packed.coeff_scale.reshape(-1) if packed.coeff_quantized else None
        basis = packed.basis.to(device=packed.device)
        out = kernels.c1_restore(coeff.to(packed.device), scale, basis, packed.original_dtype)
        return out.reshape(packed.original_shape)

    # ---------------------------------------------------------------- statistics
    def stats(self) -> Dict[str, Any]:
        first = self._first_nonfinite_event or {}
        out: Dict[str, Any] = {
            "site_id": self.spec.site_id, "module_type": self.spec.module_type,
            "hidden_size": self.spec.hidden_size, "rank": self.spec.rank,
            "pack_count": self.pack_count, "unpack_count": self.unpack_count,
            "compressed_pack_count": self._count("_compressed_pack_count"),
            "duplicate_pack_count": self._count("_duplicate_pack_count"),
            "fallback_count": self._count("_fallback_count"),
            "basis_refresh_count": self.basis_refresh_count, "step_count": self.step_count,
            "basis_initialized": self.basis_initialized, "basis_dtype": _dtype_name(self.basis.dtype),
            "energy_ewma": float(self._energy_ewma.item()), "last_energy": float(self._last_energy.item()),
            "warmup_steps": self.spec.warmup_steps,
            "refresh_energy_threshold": float(self.spec.refresh_energy_threshold),
            "raw_bytes_total": self._count("_raw_bytes_total"),
            "stored_bytes_total": self._count("_stored_bytes_total"),
            "basis_persistent_bytes": self.basis.numel() * self.basis.element_size(),
            "basis_init_refresh_count": self._count("_basis_init_refresh_count"),
            "basis_warmup_refresh_count": self._count("_basis_warmup_refresh_count"),
            "basis_trigger_refresh_count": self._count("_basis_trigger_refresh_count"),
            "fallback_reasons": dict(self._fallback_reasons),
        }
        for key in ("step", "reason", "stage"):
            out[f"first_nonfinite_{key}"] = first.get(key)
        for key in ("input", "coeff", "reconstruction", "residual", "basis"):
            out[f"first_nonfinite_{key}_max_abs"] = first.get(f"{key}_max_abs")
        for key in ("input", "coeff", "reconstruction", "residual", "basis"):
            out[f"last_{key}_max_abs"] = self._last[key]
        return out


def serialize_packed_record(record: CompressedBoundaryRecord) -> Tuple[Dict[str, Any], list]:
    """(metadata, tensors) of a record, for the checkpoint function's saved state (:759-782)."""
    if record.is_dense_fallback:
        assert record.dense_tensor is not None
        tensors = [record.dense_tensor]
    else:
        assert record.coeff is not None and record.basis is not None
        tensors = [record.coeff] + ([record.coeff_scale] if record.coeff_scale is not None else []) + [record.basis]
    meta = {"site_id": record.site_id, "original_shape": tuple(record.original_shape),
            "original_dtype": record.original_dtype, "device": record.device,
            "is_dense_fallback": record.is_dense_fallback, "coeff_quantized": record.coeff_quantized,
            "has_coeff_scale": record.coeff_scale is not None}
    return meta, tensors


def deserialize_packed_record(meta: Dict[str, Any], tensors) -> CompressedBoundaryRecord:
    """The record serialize_packed_record describes (:785-810)."""
    head = (meta["site_id"], tuple(meta["original_shape"]), meta["original_dtype"], meta["device"])
    if meta["is_dense_fallback"]:
        return CompressedBoundaryRecord(*head, True, dense_tensor=tensors[0])
    has_scale = bool(meta.get("has_coeff_scale"))
    return CompressedBoundaryRecord(*head, False, coeff=tensors[0], coeff_scale=tensors[1] if has_scale else None,
                                    coeff_quantized=bool(meta.get("coeff_quantized", False)),
                                    basis=tensors[2 if has_scale else 1])


# the reference's module-private names
_serialize_packed_record = serialize_packed_record
_deserialize_packed_record = deserialize_packed_record

__all__ = ["STACRCheckpointSpec", "CompressedBoundaryRecord", "CheckpointBoundaryCodec", "serialize_packed_record",
           "deserialize_packed_record"]
