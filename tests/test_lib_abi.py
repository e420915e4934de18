"""The C-ABI library loads, exports every symbol ``include/mosaic_amd.h``
declares, and validates arguments on the host (no GPU call is made)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "mosaic_amd.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mosaic_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from mosaic_amd import _lib

    if not _lib.LIB_PATH.exists():
        from mosaic_amd.build import build

        build()
    return _lib.lib()


def test_every_declared_symbol_is_exported_and_bound(lib):
    from mosaic_amd import _lib

    names = _declared()
    assert len(names) >= 14
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/mosaic_amd.h but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature in mosaic_amd/_lib.py"
    assert set(_lib.SIGNATURES) <= set(names)


def test_version_matches_header(lib):
    m = re.search(r"#define MOSAIC_AMD_ABI_VERSION (\d+)", HEADER.read_text())
    assert lib.mosaic_version() == int(m.group(1))


def test_invalid_arguments_are_rejected_on_the_host(lib):
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rc = lib.mosaic_mx_linear_a16(p, p, p, p, 1, 16, 100, None)
    assert rc < 0
    assert b"multiple of 128" in lib.mosaic_last_error()
    rc = lib.mosaic_mx_quantize(p, 0, p, p, 4, 33, 0, None)
    assert rc < 0 and b"multiple of 32" in lib.mosaic_last_error()
    rc = lib.mosaic_moe_route_topk(p, 1, 600, 8, 0, 1, 1.0, None, p, p, None)
    assert rc < 0 and b"E=600" in lib.mosaic_last_error()
    rc = lib.mosaic_mxt16_prepack(p, p, p, p, 24, 128, None)
    assert rc < 0 and b"multiple of 16" in lib.mosaic_last_error()


def test_python_wrappers_reject_cpu_tensors():
    import torch

    from mosaic_amd import ops

    with pytest.raises(ValueError, match="GPU tensor"):
        ops.mx_linear_a16(torch.zeros(1, 128, dtype=torch.bfloat16), torch.zeros(16, 64, dtype=torch.uint8),
                          torch.zeros(16, 4, dtype=torch.uint8))
