"""The library loads in a process before or after PyTorch.  It links no ROCm library that
PyTorch ships a different build of (rocBLAS, hipBLASLt): when the matrix prefill used rocBLAS,
loading this library and then importing torch crashed the process."""

import subprocess
import sys
from pathlib import Path

import pytest

LIB = Path(__file__).resolve().parents[1] / "tiles_amd" / "libtileinfer_amd.so"


@pytest.mark.parametrize("torch_first", [False, True])
def test_library_and_torch_load_in_either_order(torch_first):
    if not LIB.exists():
        pytest.skip("library not built")
    load = f"ctypes.CDLL({str(LIB)!r}, mode=os.RTLD_NOW | ctypes.RTLD_GLOBAL)"
    steps = ["import torch", load] if torch_first else [load, "import torch"]
    code = "; ".join(["import ctypes, os", *steps, "print('ok')"])
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0 and out.stdout.strip() == "ok", (out.returncode, out.stderr[-500:])
