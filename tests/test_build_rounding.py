"""The separately rounded f32 helpers (cea_common.hpp: mul_rn / add_rn) keep the reference's
rounding points even in translation units compiled with FMA contraction on (the attention,
decode and merge kernels are): a merge written as add_rn(mul_rn(a, w), mul_rn(b, v)) — the
reference's ``out_a * w_a + out_b * w_b`` in f32 tensor ops (attention.py:242-264) — must
compile to two multiplies and an add, never to a fused multiply-add.  Checked on the gfx950
assembly that the package's own compile flags produce (hipcc cross-compiles without a GPU).
"""

from __future__ import annotations

import importlib
import re
import shutil
import subprocess

import pytest

build = importlib.import_module("collaborative-edge-system_amd.build")

SNIPPET = r"""
#include "cea_common.hpp"
__global__ void merge_two(const float* a, float* o) {
  const int i = threadIdx.x;
  o[i] = cea::add_rn(cea::mul_rn(a[i], a[i + 64]), cea::mul_rn(a[i + 128], a[i + 192]));
}
__global__ void merge_two_f64(const double* a, double* o) {
  const int i = threadIdx.x;
  o[i] = cea::add_rn(cea::mul_rn(a[i], a[i + 64]), cea::mul_rn(a[i + 128], a[i + 192]));
}
"""


def _asm(tmp_path, extra):
    src = tmp_path / "rounding.hip"
    src.write_text(SNIPPET)
    out = tmp_path / "rounding.s"
    flags = [f for f in build.COMMON_FLAGS if f not in ("-fPIC",)]
    cmd = [build.HIPCC, *flags, *extra, "--cuda-device-only", "-S", str(src), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=300)
    return out.read_text()


def _body(asm: str, mangled: str) -> str:
    m = re.search(rf"^{mangled}:(.*?)s_endpgm", asm, re.S | re.M)
    assert m, f"kernel {mangled} not found in the assembly"
    return m.group(1)


@pytest.mark.skipif(shutil.which(build.HIPCC) is None and not build.HIPCC.startswith("/"),
                    reason="hipcc not available")
@pytest.mark.parametrize("contract", ["", "fast-honor-pragmas", "on", "off"],
                         ids=["hip-default", "fast-honor-pragmas", "on", "off"])
def test_rounded_helpers_never_fuse(tmp_path, contract):
    """HIP's default contraction mode (fast-honor-pragmas, what the attention, decode and
    merge kernels build with) and the stricter ones.  Plain -ffp-contract=fast lets the
    backend fuse regardless of the helpers' pragma; no file of the package builds with it."""
    asm = _asm(tmp_path, [f"-ffp-contract={contract}"] if contract else [])
    for name, fma in (("_Z9merge_twoPKfPf", r"v_fma\w*_f32|v_fmac\w*_f32"),
                      ("_Z13merge_two_f64PKdPd", r"v_fma\w*_f64")):
        body = _body(asm, name)
        assert not re.search(fma, body), f"{name}: fused multiply-add under -ffp-contract={contract}"
        assert len(re.findall(r"v_mul_f(32|64)", body)) >= 2, f"{name}: expected two multiplies"
