"""The fp8 quantiser's corrected quotient (ltx_common.h, quotient_e4m3_corrected)
gives the e4m3 code of the IEEE quotient x / scale for every bf16 input and
every bf16 frame maximum at or above 2^-96: an exhaustive C check over all
such pairs (about 9e8), plus the C check's e4m3 encoder pinned against
torch's float8_e4m3fn cast on the values that decide rounding (every e4m3
midpoint and its float32 neighbours, the subnormal range, the clamp)."""
import os
import shutil
import subprocess

import numpy as np
import pytest
import torch

SRC = os.path.join(os.path.dirname(__file__), "native", "e4m3_corrected_quotient.c")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = str(tmp_path_factory.mktemp("e4m3") / "check")
    subprocess.run([gcc, "-O2", "-fopenmp", "-ffp-contract=off", "-o", exe, SRC, "-lm"], check=True)
    return exe


def _decision_values():
    """Every e4m3 value, every midpoint between neighbours, the float32
    neighbours of both, and a sweep of the subnormal range."""
    codes = torch.arange(0, 0x7F, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()  # 0 .. 448
    mids = (codes[:-1] + codes[1:]) / 2
    pts = np.concatenate([codes, mids]).astype(np.float32)
    nb = np.concatenate([pts, np.nextafter(pts, np.float32(np.inf)), np.nextafter(pts, np.float32(0))])
    sub = np.linspace(0, 2 ** -6, 4097, dtype=np.float32)
    big = np.array([448, 449, 463.99, 464, 480, 1e6], dtype=np.float32)
    v = np.concatenate([nb, sub, big])
    return np.concatenate([v, -v]).astype(np.float32)


def test_encoder_matches_torch_cast(checker):
    v = _decision_values()
    out = subprocess.run([checker, "encode"], input="\n".join(repr(float(x)) for x in v),
                         capture_output=True, text=True, check=True).stdout.split()
    got = np.array([int(c) for c in out], dtype=np.uint8)
    ref = torch.from_numpy(np.clip(v, -448, 448)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert got.shape == ref.shape
    assert (got == ref).all(), v[got != ref][:8]


@pytest.mark.timeout(600)
def test_corrected_quotient_codes_equal_division_exhaustive(checker):
    res = subprocess.run([checker], capture_output=True, text=True)
    print(res.stdout)
    words = res.stdout.split()
    pairs, codes = int(words[1]), int(words[5])
    assert pairs > 9 * 10 ** 8
    assert codes == 0 and res.returncode == 0
