"""CPU checks of the C-ABI boundary: the library builds/loads and exports every
symbol include/flashrec_amd.h declares, the ctypes table matches the header,
and the Python mirror refuses CPU tensors instead of falling back."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "flashrec_amd.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|int64_t)\s+(fr_\w+)\s*\(", text, flags=re.M)))


def _declared_arity():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for name, args in re.findall(r"^(?:int|int64_t)\s+(fr_\w+)\s*\(([^)]*)\)", text, flags=re.M | re.S):
        args = args.strip()
        out[name] = 0 if args in ("", "void") else len(args.split(","))
    return out


def test_library_exports_every_declared_symbol():
    from flashrec_amd import _lib

    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    names = _declared()
    assert len(names) >= 12
    for name in names:
        assert hasattr(lib, name), f"{name} declared but not exported"
    assert lib.fr_abi_version() == 1


def test_ctypes_table_matches_header():
    from flashrec_amd import _lib

    arity = _declared_arity()
    assert set(arity) == set(_lib.SIGNATURES)
    for name, n in arity.items():
        assert len(_lib.SIGNATURES[name]) == n, name


def test_invalid_arguments_rejected_without_gpu():
    """Argument validation happens before any launch, so it runs on a CPU host."""
    from flashrec_amd import _lib

    lib = _lib.load()
    # null pointers with a non-empty shape
    assert lib.fr_per_token_quant_fp8(None, 0, 4, 8, 8, None, None, None) == _lib.FR_EINVAL
    assert lib.fr_fp8_scaled_mm(None, 16, None, 16, None, 1, None, 1, None, 0, None, 4, 4, 4, 16, 0,
                                None) == _lib.FR_EINVAL
    # negative sizes
    assert lib.fr_silu_quant_fp8(None, 0, 0, -1, 4, None, None, None) == _lib.FR_EINVAL
    # unsupported head dim
    args = [None] * 28
    args[25] = 256
    for i in (1, 2, 4, 5, 7, 8, 15, 17, 18, 20, 21, 22, 23, 24):
        args[i] = 1
    args[13] = 1e-6
    args[26] = 1
    args[27] = None
    args[23] = 1
    args[24] = 1
    assert lib.fr_qk_norm_rope_store_fp8(*args) == _lib.FR_EUNSUPPORTED
    # empty work is a no-op success
    assert lib.fr_per_token_quant_fp8(None, 0, 0, 8, 8, None, None, None) == _lib.FR_OK


@pytest.mark.parametrize("fn", ["per_token_quant_fp8", "silu_and_mul", "rmsnorm"])
def test_cpu_tensors_raise(fn):
    from flashrec_amd.kernel import sglops

    x = torch.zeros(2, 8, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU path"):
        if fn == "rmsnorm":
            sglops.rmsnorm(x, torch.ones(8), 1e-6)
        else:
            getattr(sglops, fn)(x)


def test_fused_ops_raise_on_cpu():
    from flashrec_amd.kernel.rms_fp8 import rmsnorm_per_token_quant_fp8
    from flashrec_amd.kernel.silu_fp8 import silu_and_mul_per_token_quant_fp8

    x = torch.zeros(2, 8, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU path"):
        rmsnorm_per_token_quant_fp8(x, torch.ones(8), 1e-6)
    with pytest.raises(RuntimeError, match="no CPU path"):
        silu_and_mul_per_token_quant_fp8(x)


def test_product_does_not_import_oracle():
    for p in (ROOT / "flashrec_amd").rglob("*.py"):
        assert "oracle" not in re.findall(r"^\s*(?:from|import)\s+(\w+)", p.read_text(), flags=re.M), p


def test_header_constants_match_the_library_sources():
    """Status codes and capacities are defined in the public header and in the
    kernels' common header: both, and the Python binding, must agree."""
    from flashrec_amd import _lib

    def defines(path):
        text = (ROOT / path).read_text()
        return {m.group(1): m.group(2).strip() for m in re.finditer(r"#define (FR_\w+) (.+?)(?:\s*/[*/].*)?$",
                                                                     text, re.M)}

    pub = defines("include/flashrec_amd.h")
    kern = defines("flashrec_amd/csrc/fr_common.h")
    for name in ("FR_OK", "FR_EINVAL", "FR_EUNSUPPORTED", "FR_ELAUNCH", "FR_ETOOLARGE",
                 "FR_GENREC_NOALLOC_SCRATCH_BYTES", "FR_DTYPE_BF16", "FR_DTYPE_E4M3"):
        assert pub[name] == kern[name], name
    assert int(pub["FR_ETOOLARGE"]) == _lib.FR_ETOOLARGE
    assert eval(pub["FR_GENREC_NOALLOC_SCRATCH_BYTES"]) == _lib.GENREC_NOALLOC_SCRATCH_BYTES
