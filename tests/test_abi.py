"""ABI conformance on the CPU: the provider's header and its Python mirror
have the reference waist's exact layouts (neuro_fabric_abi.h:148-162,
neuro_buffer_abi.h:94-216, neuro_scheduler_abi.h:86-127, neuro_ddi.h:33-76)."""
import subprocess
from pathlib import Path

import pytest

from neurofabric_amd import abi

REPO = Path(__file__).resolve().parents[1]

PROBE = r"""
#include <stddef.h>
#include <stdio.h>
#include "nf_abi.h"
#include "nf_hip_plugin.h"
int main(void) {
  printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu %u\n",
         sizeof(nf_tensor_desc), sizeof(nf_buffer_info), sizeof(nf_buffer_alloc_request),
         sizeof(nf_task_desc), sizeof(nf_driver_caps), sizeof(nf_push_constants),
         offsetof(nf_task_desc, inputs), offsetof(nf_task_desc, push_constants),
         offsetof(nf_push_constants, M), (unsigned)NF_ABI_VERSION);
  return 0;
}
"""


def test_python_mirror_layout():
    abi.check_layout()


@pytest.mark.parametrize("compiler,std,ext", [("gcc", "-std=c11", "c"), ("g++", "-std=c++17", "cpp")])
def test_header_compiles_with_pinned_layout(tmp_path, compiler, std, ext):
    src = tmp_path / f"probe.{ext}"
    src.write_text(PROBE)
    exe = tmp_path / "probe"
    subprocess.run([compiler, std, "-Wall", "-Werror", f"-I{REPO / 'include'}", str(src), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    assert out == ["144", "176", "160", "3056", "32", "48", "64", "2988", "20", str(0x000200)]


def test_status_and_dtype_values():
    assert (abi.NF_OK, abi.NF_ERROR_INVALID_ARG, abi.NF_ERROR_UNSUPPORTED_OP,
            abi.NF_ERROR_DEVICE_LOST, abi.NF_ERROR_TIMEOUT, abi.NF_ERROR_INTERNAL) == (0, 1, 7, 6, 8, 255)
    assert (abi.NF_DTYPE_F32, abi.NF_DTYPE_F16, abi.NF_DTYPE_Q4_0, abi.NF_DTYPE_Q8_0) == (0, 1, 6, 7)
    assert abi.NF_ABI_VERSION == 0x000200
