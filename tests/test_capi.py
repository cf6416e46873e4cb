"""CPU: the C-ABI library loads, exports every entry point declared in
include/scope_amd.h, and the ctypes structs match the C layouts (checked by
compiling the header with gcc).  No compute calls are made here."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "scope_amd.h")
LIB = os.path.join(ROOT, "scope_amd", "libscope_amd.so")


def declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(scope_[a-z0-9_]+)\s*\(", text)))


needs_lib = pytest.mark.skipif(not os.path.exists(LIB), reason="libscope_amd.so not built")


@needs_lib
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    names = declared_functions()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


@needs_lib
def test_abi_version_and_error_string():
    from scope_amd import _lib

    lib = _lib.load()
    assert lib.scope_abi_version() == _lib.ABI_VERSION
    assert isinstance(lib.scope_last_error(), bytes)


@needs_lib
def test_prototypes_cover_header():
    from scope_amd import _lib

    assert sorted(_lib._PROTOS) == declared_functions()


def test_ctypes_struct_layouts_match_c():
    from scope_amd._lib import (AttnParams, CoeffParams, DecodeParams, MlpParams, PtrBwdParams, PtrRefParams,
                                PtrScoreParams, StatsParams, WgradParams)

    structs = {"scope_ptr_ref_params": PtrRefParams, "scope_ptr_score_params": PtrScoreParams,
               "scope_stats_params": StatsParams, "scope_attn_params": AttnParams,
               "scope_ptr_bwd_params": PtrBwdParams, "scope_coeff_params": CoeffParams,
               "scope_decode_params": DecodeParams, "scope_wgrad_params": WgradParams,
               "scope_mlp_params": MlpParams}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0; }")
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "layout.c"), os.path.join(d, "layout")
        open(src, "w").write("\n".join(lines))
        subprocess.run(["gcc", "-std=c11", src, "-o", exe], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split("\n")
    got = dict(line.rsplit(" ", 1) for line in out if line)
    for cname, cls in structs.items():
        assert int(got[f"{cname} size"]) == ctypes.sizeof(cls), cname
        for fname, _ in cls._fields_:
            assert int(got[f"{cname}.{fname}"]) == getattr(cls, fname).offset, f"{cname}.{fname}"


def test_ops_refuse_cpu_tensors():
    """No CPU fallback: every op raises before touching the library."""
    import torch

    from scope_amd import ops

    docs = torch.zeros(256, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.doc_starts(docs, 128)
    q = torch.zeros((1, 2, 256, 128), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.block_means(q, q, 128)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.attn_fwd(q, q, q, torch.ones((2, 2), dtype=torch.int32), torch.zeros((2, 2, 1), dtype=torch.int32),
                     docs, torch.zeros(2, dtype=torch.int32), bs=128, scale=0.12)
    # the decoder's token-step ops
    x = torch.zeros(1024, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.decoder_gemv(x, torch.zeros((8, 1024), dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="GPU"):
        ops.argmax(torch.zeros(10))
    i1 = torch.zeros(1, dtype=torch.int64)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.decoder_step_prologue(i1, i1, torch.zeros(8, dtype=torch.int64), torch.zeros(8, dtype=torch.int32),
                                  torch.zeros((4, 1024), dtype=torch.bfloat16), [], eot=3)


def test_missing_library_raises(tmp_path):
    from scope_amd import _lib

    with pytest.raises(_lib.ScopeLibraryError, match="not found"):
        _lib.load(str(tmp_path / "nope.so"))
