"""CPU checks of the C-ABI library: it loads, exports every symbol that
include/yuuka_hip.h declares, and reports ABI version 10 (reference
RequiredABI, backend/hip/hip.go:49). No device calls."""
import subprocess

from yuuka_amd import hip


def test_library_exports_every_declared_symbol():
    names = hip.header_symbols()
    assert len(names) >= 45
    L = hip.lib()
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    dyn = subprocess.run(["nm", "-D", "--defined-only", str(hip.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in dyn.splitlines() if line.strip()}
    assert set(names) <= exported


def test_abi_versions_and_empty_error():
    assert hip.lib().yuuka_abi_version() == 10
    assert hip.lib().yuuka_ext_version() == 1
    assert hip.lib().yuuka_last_error() in (b"",)


def test_quantized_bytes_rules():
    assert hip.quantized_bytes(2560, 5) == 64 + 2560 * 17
    assert hip.quantized_bytes(2560, 9) == 64 + 2 * 2560 * 17
    assert hip.quantized_bytes(100, 5) == 0 and hip.quantized_bytes(256, 17) == 0
