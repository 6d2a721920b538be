"""GPU parity of the mixed-precision quantizers (qkv_compress_mixed /
qkv_decompress_mixed) against the reference's golden vectors and the CPU
oracle: codes from identical rotated inputs bit-exact, codes from x equal to
the golden ones, reconstructions to 1e-5."""

import numpy as np
import pytest
import torch

import quashkv_amd as Q
from quashkv_amd import _native as N
from oracle import ref_math as R

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    N.lib()


def T(a):
    return torch.from_numpy(np.asarray(a))


def test_mixed_mse_vs_golden(golden):
    g = golden("mixed")
    qm = Q.MixedPrecisionMSEQuantizer(128, outlier_bits=3, regular_bits=2, n_outliers=32,
                                      seed=42, device=DEV)
    qm.calibrate(T(g["calib"]).to(DEV))
    assert torch.equal(qm._outlier_indices.cpu(), T(g["outliers"]))
    assert qm.effective_bits == 2.25
    codes, norms = qm.compress(T(g["x"]).to(DEV))
    assert codes.shape == (3, 2, 8, 128) and codes.dtype == torch.uint8
    assert torch.equal(codes.cpu(), T(g["idx"]))
    assert torch.allclose(norms.cpu(), T(g["norm"]), rtol=1e-6)
    xh = qm.decompress(codes, norms)
    assert torch.allclose(xh.cpu(), T(g["xhat"]), rtol=1e-5, atol=1e-5)
    # uncalibrated: the regular codebook everywhere
    qm2 = Q.MixedPrecisionMSEQuantizer(64, outlier_bits=4, regular_bits=2, n_outliers=8,
                                       seed=43, device=DEV)
    c2, n2 = qm2.compress(T(g["x2"]).to(DEV))
    assert torch.equal(c2.cpu(), T(g["idx2"]))
    assert torch.allclose(qm2.decompress(c2, n2).cpu(), T(g["xhat2"]), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("d,ob,rb,no", [(128, 3, 2, 32), (64, 4, 2, 8), (96, 4, 3, 20)])
def test_mixed_codes_from_identical_y_bit_exact(d, ob, rb, no):
    gen = torch.Generator().manual_seed(d + ob)
    qm = Q.MixedPrecisionIPQuantizer(d, outlier_bits=ob, regular_bits=rb, n_outliers=no,
                                     seed=5, device=DEV)
    out_idx = torch.randperm(d, generator=gen)[:no]
    qm.set_outlier_channels(out_idx.to(DEV))
    mq = qm.mse_quantizer
    y = torch.randn(500, d, generator=gen) / d ** 0.5
    y[7, 3] = float(mq.regular_codebook.boundaries[0])    # exact ties
    y[9, out_idx[0]] = float(mq.outlier_codebook.boundaries[1])
    codes = qm._quantize_mixed(y.to(DEV)).cpu()
    mask = torch.zeros(d, dtype=torch.bool)
    mask[out_idx] = True
    ref = torch.where(mask, R.quantize_boundary(y, mq.outlier_codebook.boundaries.cpu()),
                      R.quantize_boundary(y, mq.regular_codebook.boundaries.cpu()))
    assert torch.equal(codes, ref)


@pytest.mark.parametrize("d", [64, 128])
def test_mixed_ip_compress_vs_oracle(d):
    gen = torch.Generator().manual_seed(d)
    qm = Q.MixedPrecisionIPQuantizer(d, outlier_bits=4, regular_bits=3, n_outliers=d // 4,
                                     seed=11, device=DEV)
    calib = torch.randn(2048, d, generator=gen)
    calib[:, :4] *= 5
    qm.calibrate(calib.to(DEV))
    x = torch.randn(64, 3, d, generator=gen)
    mse, qjl, norms = qm.compress(x.to(DEV))
    mq = qm.mse_quantizer
    pi, oi = mq.Pi.cpu(), mq._outlier_indices.cpu()
    ref_codes, ref_norms = R.mixed_compress(x, pi, oi, mq.outlier_codebook.boundaries.cpu(),
                                            mq.regular_codebook.boundaries.cpu())
    assert float((mse.cpu() != ref_codes).double().mean()) <= 1e-3
    # QJL sign of the residual against each channel's centroid, on the same codes
    y = (x / ref_norms.unsqueeze(-1)) @ pi.T
    mask = torch.zeros(d, dtype=torch.bool)
    mask[oi] = True
    cent = torch.where(mask, mq.outlier_codebook.centroids.cpu()[mse.cpu().long().clamp(max=15)],
                       mq.regular_codebook.centroids.cpu()[
                           mse.cpu().long().clamp(max=mq.regular_codebook.n_levels - 1)])
    ref_bits = (((y - cent) * qm.S.cpu()) >= 0).to(torch.uint8)
    assert float((qjl.cpu() != ref_bits).double().mean()) <= 1e-3
    assert torch.allclose(norms.cpu(), ref_norms, rtol=1e-6)
    deq = qm._dequantize_mixed(mse)
    assert torch.allclose(deq.cpu(), cent, rtol=0, atol=0)
