"""The library's fp32 -> bf16 rounding (gfx950's packed conversion, pk_device.h) gives
the integer round-to-nearest-even bits for every one of the 2^32 fp32 inputs, NaNs
included (tests/native/bf16_rounding_check.hip, built by parakeet-streaming_amd/build.py)."""
import subprocess
from pathlib import Path

import pytest

EXE = Path(__file__).resolve().parent / "native" / "_build" / "bf16_rounding_check"


@pytest.mark.gpu
def test_bf16_rounding_matches_integer_rne_for_every_fp32():
    if not EXE.exists():
        raise RuntimeError(f"{EXE} is missing: build it with parakeet-streaming_amd/build.py")
    print(f"running {EXE.name}", flush=True)
    res = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=90)
    assert res.returncode == 0 and "mismatches 0 " in res.stdout, (res.returncode, res.stdout, res.stderr)
