"""Write the golden vectors of MixedPrecisionIPQuantizer.compress.

Like make_golden.py, this runs ONLY in the build container, where the
reference package is mounted read-only (default ``/root/reference``): it
imports the reference, feeds its mixed-precision IP quantizer
(``quashkv/mixed_precision.py:200-322``) small seeded inputs and stores inputs
and outputs in ``mixed_ip.npz`` next to this script.  The per-channel MSE
codes alone are pinned by ``mixed.npz`` and the QJL rule alone by
``compress.npz``; these vectors pin their combination (the residual taken
against each channel's own codebook).

Usage:  python tests/golden/make_golden_mixed_ip.py [--ref /root/reference]
"""

from __future__ import annotations

import argparse
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def _np(t):
    return t.detach().cpu().numpy()


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    args = ap.parse_args()

    sys.dont_write_bytecode = True
    sys.path.insert(0, args.ref)
    import torch  # noqa: E402

    torch.set_num_threads(4)
    import quashkv

    assert os.path.abspath(quashkv.__file__).startswith(os.path.abspath(args.ref)), quashkv.__file__
    from quashkv.mixed_precision import MixedPrecisionIPQuantizer

    out = {}
    g = torch.Generator().manual_seed(77)
    # (tag, d, outlier_bits, regular_bits, n_outliers, seed, calibrated)
    cases = (("a", 128, 3, 2, 32, 42, True), ("b", 128, 3, 2, 64, 43, True),
             ("c", 64, 4, 3, 16, 44, True), ("d", 64, 3, 2, 16, 45, False))
    for tag, d, ob, rb, n_out, seed, calibrated in cases:
        q = MixedPrecisionIPQuantizer(d, outlier_bits=ob, regular_bits=rb, n_outliers=n_out,
                                      seed=seed)
        scale = torch.ones(d)
        scale[torch.randperm(d, generator=g)[:n_out]] = 6.0
        if calibrated:
            calib = torch.randn(2048, d, generator=g)
            # outlier channels of the rotated space: scale there, rotate back
            pi = q.mse_quantizer.Pi
            calib = (calib * scale) @ pi
            q.calibrate(calib)
            out[f"{tag}_outliers"] = _np(q.mse_quantizer._outlier_indices)
        x = ((torch.randn(4, 3, 16, d, generator=g) * scale) @ q.mse_quantizer.Pi)
        codes, bits, norms = q.compress(x)
        out[f"{tag}_x"] = _np(x)
        out[f"{tag}_codes"] = _np(codes)
        out[f"{tag}_qjl"] = _np(bits)
        out[f"{tag}_norm"] = _np(norms)
        out[f"{tag}_S"] = _np(q.S)
        out[f"{tag}_cfg"] = np.array([d, ob, rb, n_out, seed, int(calibrated)], dtype=np.int64)
    np.savez_compressed(os.path.join(HERE, "mixed_ip.npz"), **out)
    print("mixed_ip done")


if __name__ == "__main__":
    main()
