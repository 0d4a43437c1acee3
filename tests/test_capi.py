"""The C-ABI library loads, exports every declared symbol, and its host-only
parts (parser, host erff) work without a GPU."""
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "shlo_hip.h")).read()
    return sorted(set(re.findall(r"\b(shlo_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_symbol():
    import shlo_hip
    lib = shlo_hip.lib_handle()
    names = _declared()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert missing == []


def test_reference_boundary_is_covered():
    """One shlo_* per smlx_* of the reference shim (c/smlx_shim.c)."""
    smlx = ["empty", "of_bytes", "to_bytes", "shape", "dtype", "unary", "binary", "where", "reshape",
            "transpose", "broadcast", "slice", "concat", "astype", "view", "take", "max_axis", "contiguous",
            "eval", "kernel_new", "kernel_apply", "compile", "apply", "libm_erff_range", "count_nonzero"]
    assert len(smlx) == 25
    names = set(_declared())
    assert [s for s in smlx if "shlo_" + s not in names] == []


MODULE = """module @m attributes {mhlo.frontend_attributes = {}} {
  // a comment
  func.func public @main(%a0: tensor<2x3xf32>, %a1: tensor<3x2xf32> {jax.arg = "x"}) -> (tensor<2x2xf32>) {
    %0 = "stablehlo.dot_general"(%a0, %a1) {dot_dimension_numbers = #stablehlo.dot<lhs_contracting_dimensions = [1], rhs_contracting_dimensions = [0]>} : (tensor<2x3xf32>, tensor<3x2xf32>) -> tensor<2x2xf32>
    %1:2 = "stablehlo.custom_call"(%0) {call_target_name = "x"} : (tensor<2x2xf32>) -> (tensor<2x2xf32>, tensor<2x2xf32>)
    func.return %1#0 : tensor<2x2xf32>
  }
}
"""


def test_parse_and_arg_types():
    import shlo_hip
    m = shlo_hip.Module(MODULE)
    assert m.arg_types() == [((2, 3), shlo_hip.F32), ((3, 2), shlo_hip.F32)]


@pytest.mark.parametrize("text,msg", [
    ("module { func.func @f() { } }", "no @main"),
    ("module { func.func @main() { %0 = stablehlo.add %a, %b : tensor<f32> } }", "unsupported op syntax"),
    ("module { func.func @main() { } } trailing", "trailing text"),
])
def test_parse_errors(text, msg):
    import shlo_hip
    with pytest.raises(shlo_hip.ShloError, match=msg):
        shlo_hip.Module(text)


def test_unknown_kernel_refused():
    import shlo_hip
    with pytest.raises(shlo_hip.ShloError, match="no precompiled kernel"):
        shlo_hip.Kernel("nope")
    assert shlo_hip.Kernel("smlx_mul_mat") is not None


def test_host_erff_spot_values():
    import shlo_hip
    out = shlo_hip.libm_erff_range(0x3F800000, 1)  # erf(1)
    assert out[0] == 0x3F57BB3D
    assert shlo_hip.libm_erff_range(0x7F800000, 1)[0] == 0x3F800000   # +inf -> 1
    assert shlo_hip.libm_erff_range(0xFF800000, 1)[0] == 0xBF800000   # -inf -> -1
    assert shlo_hip.libm_erff_range(0x80000000, 1)[0] == 0x80000000   # -0 -> -0
    assert shlo_hip.libm_erff_range(0x7FC00001, 1)[0] == 0x7FC00001   # NaN -> NaN quieted, payload kept
