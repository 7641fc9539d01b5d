"""The C-ABI library loads and exports every symbol include/fast_mimi_amd.h
declares (no kernel is launched here: this suite runs without a GPU)."""

from __future__ import annotations

import re
import subprocess

import pytest

from conftest import REPO
from fast_mimi_amd import _native as nat

HEADER = REPO / "include" / "fast_mimi_amd.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t)\s+(fm_\w+)\s*\(", text, re.M)))


def test_header_declares_the_bound_entry_points():
    assert declared_symbols() == sorted(nat.exported_symbols())


def test_library_exports_every_declared_symbol():
    if not nat.LIBRARY_PATH.is_file():
        pytest.skip("library not built")
    lib = nat.library()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(nat.LIBRARY_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (fm_\w+)", out))
    assert set(declared_symbols()) <= exported
    assert lib.fm_abi_version() == nat.ABI_VERSION


def test_workspace_query_is_host_only():
    if not nat.LIBRARY_PATH.is_file():
        pytest.skip("library not built")
    lib = nat.library()
    a = lib.fm_rvq_workspace_bytes(125, 256, 2048)
    b = lib.fm_rvq_workspace_bytes(250, 256, 2048)
    assert 0 < a < b


def test_status_codes_map_to_errors():
    with pytest.raises(nat.NativeError, match="bad argument"):
        nat.check(1000, "fm_x")
    with pytest.raises(nat.NativeError, match="hipError_t 700"):
        nat.check(700, "fm_x")
    nat.check(0, "fm_x")


def test_torch_ops_mirror_the_header():
    """Every stream-taking entry point is a torch.ops.fast_mimi_amd operator
    whose schema follows the C signature (stream dropped; const pointers
    read-only, other pointers mutated)."""
    import torch

    from fast_mimi_amd import ops

    text = HEADER.read_text()
    for ret, name, args in re.findall(r"^\s*(int|size_t)\s+(fm_\w+)\s*\(([^)]*)\)", text, re.M):
        params = [a.strip() for a in args.replace("\n", " ").split(",") if a.strip() not in ("", "void")]
        if not params or not params[-1].startswith("hipStream_t"):
            continue
        schema = getattr(torch.ops.fast_mimi_amd, name[3:]).default._schema
        assert len(schema.arguments) == len(params) - 1, name
        for arg, param in zip(schema.arguments, params[:-1]):
            cname = re.split(r"[\s*]+", param)[-1]
            assert arg.name == cname, (name, arg.name, cname)
            if "*" in param:
                assert str(arg.type) == "Optional[Tensor]", (name, cname)
                mutable = arg.alias_info is not None and arg.alias_info.is_write
                assert mutable == (not param.startswith("const")), (name, cname)
        assert name in ops.SPECS


def test_torch_ops_trace_as_opaque_mutating_calls():
    """The fake implementations let FX trace the operators without a GPU."""
    import torch
    from torch.fx.experimental.proxy_tensor import make_fx

    from fast_mimi_amd import ops  # noqa: F401  (registers the operators)

    def decode(codes, embeds, out):
        torch.ops.fast_mimi_amd.rvq_decode(codes, 1, 8, 125, 1, embeds, 2048, 256, out)
        return out

    gm = make_fx(decode, tracing_mode="fake")(torch.zeros(1, 8, 125, dtype=torch.int64),
                                              torch.zeros(8, 2048, 256), torch.zeros(125, 512))
    assert "fast_mimi_amd.rvq_decode" in gm.code


def test_residual_inputs_alias_their_output():
    """Entry points that add a residual may be called with y == residual (the
    runtime's in-place LayerScale residual): the schema puts residual in y's
    alias set, read-only, so functionalization orders the update correctly."""
    import torch

    from fast_mimi_amd import ops

    names = [e for e, spec in ops.SPECS.items() if "res:residual" in spec]
    assert {"fm_linear", "fm_row_linear", "fm_row_linear_packed", "fm_conv1d"} <= set(names)
    for entry in names:
        args = {a.name: a for a in getattr(torch.ops.fast_mimi_amd, entry[3:]).default._schema.arguments}
        res, y = args["residual"].alias_info, args["y"].alias_info
        assert res is not None and not res.is_write and y.is_write, entry
        assert set(res.before_set) == set(y.before_set), entry


def test_gemm_plan_query_is_host_only():
    if not nat.LIBRARY_PATH.is_file():
        pytest.skip("library not built")
    assert isinstance(nat.last_gemm_plan(), str)
    with pytest.raises(nat.NativeError, match="bad argument"):
        nat.check(nat.library().fm_gemm_last_plan(None, 0), "fm_gemm_last_plan")
