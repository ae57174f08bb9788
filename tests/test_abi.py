"""CPU checks of the C ABI: the library loads and exports every entry point the header declares."""
import os
import re

import pytest

from exact_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    src = open(os.path.join(ROOT, "include", "exact_hip.h")).read()
    return sorted(set(re.findall(r"^(?:int|int64_t|const char\*)\s+(exact_\w+)\(", src, re.M)))


def test_header_declares_entry_points():
    names = declared()
    assert "exact_gemv_g128" in names and "exact_attention" in names and len(names) >= 20


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="library not built")
def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES or name in _lib.OTHER, name
    assert lib.exact_version() >= 100


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="library not built")
def test_header_declares_every_exported_entry_point():
    """The reverse direction: every exact_* symbol the library exports is declared in the header (and bound)."""
    import shutil
    import subprocess
    if not shutil.which("nm"):
        pytest.skip("nm not available")
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = sorted({ln.split()[-1] for ln in out.splitlines() if ln.split() and ln.split()[-1].startswith("exact_")})
    names = set(declared())
    assert [n for n in exported if n not in names] == []
    assert [n for n in exported if n not in _lib.SIGNATURES and n not in _lib.OTHER] == []


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="library not built")
def test_host_side_validation_rejects_bad_shapes_without_launching():
    """Argument checks happen on the host: null pointers and unsupported K return codes, no GPU needed."""
    lib = _lib.load()
    assert lib.exact_gemv_g128(None, 15, None, None, None, None, 1, 64, 128, None) == 1
    fake = 1 << 20   # never dereferenced: validation fails before any launch
    assert lib.exact_gemv_g128(fake, 15, fake, fake, None, fake, 1, 64, 100, None) == 2      # K % 128
    assert lib.exact_gemv_g128(fake, 9, fake, fake, None, fake, 1, 64, 128, None) == 2       # abits
    assert lib.exact_gemv_g128(fake, 15, fake, fake, None, fake, 16, 64, 128, None) == 2     # R > 15 in A16
    assert lib.exact_synth_linear(1, 2, 0, 40000, fake, fake, fake, 64, 128, 0, 64, None) == 1  # scale range
    assert lib.exact_synth_linear(1, 2, 1, 400, fake, fake, fake, 64, 128, 32, 128, None) == 2  # part offset % 64
    assert lib.exact_attention(fake, fake, fake, fake, fake, fake, fake, fake, fake, None, 1, 4, 2, 96, 64, 8192, None) == 2
    assert lib.exact_swiglu_qrow(fake, fake, fake, 15, fake, fake, None, 1, 64, 0, None, None, None) == 1   # no workspace
    assert lib.exact_swiglu_qrow(fake, fake, fake, 15, fake, fake, fake, 1, 64, 0, fake, None, None) == 1   # h aliases t
    assert lib.exact_swiglu_qrow(fake, fake, fake, 7, fake, fake, fake, 1, 64, 0, None, fake, None) == 1   # digits of int8
    assert lib.exact_gemm_g128_digits(fake, fake, fake, None, None, fake, 4, 64, 128, 0, None) == 1    # no colterm
    assert lib.exact_logits_argmax(fake, fake, None, fake, None, 1, 64, 0, None) == 1            # no workspace
    assert lib.exact_gemv(None, fake, fake, fake, 64, 128, None) == 1                            # exact::gemv: null x
    assert lib.exact_gemv(fake, fake, fake, fake, 64, 200, None) == 2                            # K % 128
    assert lib.exact_gemv(fake + 8, fake, fake, fake, 64, 128, None) == 2                        # x not 16-byte aligned
