"""The native reduced QR (stacr_qr, and stacr_qr_tall past one workgroup's registers) against
LAPACK's Householder QR on the CPU in fp64 (torch's CPU torch.linalg.qr): the same Q and R, signs
included (R[j][j] = -sign(alpha_j) * norm), Q with orthonormal columns, Q R = A, bit-identical
repeated calls, and more than 16 columns refused.
The basis refreshes that use it (orthonormalize after an Oja step) are checked in
test_gpu_oja.py and the layer tests."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    return torch.device("cuda:0")


def announce(*parts):
    print("CASE", *parts, flush=True)


def _lapack(a: torch.Tensor):
    q, r = torch.linalg.qr(a.detach().cpu().double(), mode="reduced")
    return q.numpy(), r.numpy()


def _matrix(kind: str, rows: int, cols: int, seed: int = 0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(rows, cols, generator=g)
    if kind == "near_orthonormal":  # an Oja-stepped basis: orthonormal plus a small update
        q, _ = torch.linalg.qr(a)
        a = q + 0.01 * torch.randn(rows, cols, generator=g)
    elif kind == "graded":  # columns of very different norms
        a = a * torch.logspace(0, -6, cols)
    elif kind == "zero_column":
        a[:, cols // 2] = 0.0
    elif kind == "repeated_column":
        a[:, -1] = a[:, 0]
    elif kind == "zero_below_diagonal":  # column 0 already e_0-like: dlarfg's tau = 0 branch
        a[1:, 0] = 0.0
    return a


CASES = [
    ("cfg3_c_fc_rank8", "near_orthonormal", 1024, 8),
    ("cfg3_c_proj_rank8", "near_orthonormal", 4096, 8),
    ("cfg4_up_rank16", "near_orthonormal", 2048, 16),
    ("rank16_square", "gaussian", 16, 16),
    ("rank16", "gaussian", 2048, 16),
    ("tiny", "gaussian", 5, 3),
    ("single_column", "gaussian", 777, 1),
    ("graded", "graded", 1500, 12),
    ("zero_column", "zero_column", 600, 9),
    ("repeated_column", "repeated_column", 300, 7),
    ("zero_below_diagonal", "zero_below_diagonal", 200, 5),
    ("max_elements", "gaussian", 8192, 4),
    # past 8192 elements (and in several of the cases above) the tall route: fp64 CholeskyQR with
    # LAPACK's signs, or LAPACK's Householder QR streamed through memory where columns are close to
    # dependent (the graded, zero and repeated column cases)
    ("tall_cfg4_down_rank16", "near_orthonormal", 8192, 16),
    ("tall_cfg4_rank16_32768", "gaussian", 32768, 16),
    ("tall_odd_rows", "gaussian", 8193, 4),
    ("tall_single_column", "gaussian", 40000, 1),
    ("tall_zero_below_diagonal", "zero_below_diagonal", 4096, 9),
    ("tall_graded_householder", "graded", 8192, 12),
    ("tall_zero_column_householder", "zero_column", 4096, 9),
    ("tall_repeated_column_householder", "repeated_column", 3000, 16),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_qr_matches_lapack_householder(dev, case):
    from stacr_amd import kernels

    name, kind, rows, cols = case
    announce("qr", name, rows, cols)
    a = _matrix(kind, rows, cols)
    q, r = kernels.qr(a.to(dev))
    torch.cuda.synchronize()
    q, r = q.cpu().double().numpy(), r.cpu().double().numpy()
    oq, orr = _lapack(a)
    scale = float(np.abs(orr).max())
    # R: upper triangular, within fp32 rounding of LAPACK's (signs included)
    assert np.array_equal(np.triu(r), r)
    assert np.abs(r - orr).max() <= 2e-5 * scale
    # Q: orthonormal columns (a product of reflectors, whatever A's rank), Q R = A, and where
    # LAPACK's R[j][j] is well away from zero the same column as LAPACK's (signs included)
    qq = q.T @ q
    assert np.abs(qq - np.eye(cols)).max() <= 2e-5
    assert np.abs(q @ r - a.double().numpy()).max() <= 2e-5 * scale
    well = np.abs(np.diag(orr)) > 1e-2 * scale
    assert np.abs(q[:, well] - oq[:, well]).max() <= 2e-4


def test_qr_is_deterministic_and_refuses_what_it_does_not_take(dev):
    from stacr_amd import kernels

    announce("qr determinism")
    for rows, cols, kind in ((512, 16, "gaussian"), (2048, 16, "gaussian"), (8192, 16, "near_orthonormal"),
                             (6000, 10, "graded")):
        a = _matrix(kind, rows, cols).to(dev)
        q1, r1 = kernels.qr(a)
        q2, r2 = kernels.qr(a)
        assert torch.equal(q1, q2) and torch.equal(r1, r2), (rows, cols, kind)
    with pytest.raises(NotImplementedError):
        kernels.qr(torch.randn(100, 17, device=dev))
    with pytest.raises(ValueError):
        kernels.qr(torch.randn(3, 5, device=dev))


def test_orthonormalize_uses_the_native_qr(dev):
    """oja.orthonormalize on a GPU fp32 / bf16 matrix: LAPACK's Q in the input dtype."""
    from stacr_amd import oja

    announce("orthonormalize")
    a = _matrix("near_orthonormal", 1024, 8)
    for dt in (torch.float32, torch.bfloat16):
        got = oja.orthonormalize(a.to(dev, dt))
        assert got.dtype == dt and got.shape == a.shape
        oq, _ = _lapack(a.to(dt).float())
        tol = 2e-4 if dt == torch.float32 else 8e-3
        assert np.abs(got.float().cpu().double().numpy() - oq).max() <= tol
