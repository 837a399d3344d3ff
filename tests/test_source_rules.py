"""Rules the HIP sources follow because of how the compiler treats them
(CPU only: reads the sources, and builds one probe for gfx950 with hipcc
when it is installed).

``__builtin_bit_cast`` of an element of an ext_vector_type value, written as
a bare subscript (``__builtin_bit_cast(uint32_t, acc[i])``), compiles to a
read of element 0 whatever the index (ROCm 7.2's clang: the bit cast reads
the vector's storage at its start).  A kernel that stored fp32 accumulators
that way got only the rows of element 0 right.  The sources therefore give
``__builtin_bit_cast`` rvalue operands only (a cast, an expression or a
whole value), and the probe below shows the rvalue form reading every
element.
"""

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "complexity-framework_amd" / "csrc"
BARE_SUBSCRIPT = re.compile(r"__builtin_bit_cast\(\s*[\w:]+\s*,\s*[A-Za-z_]\w*(\s*\[[^\[\]]+\])+\s*\)")


def test_no_bit_cast_of_a_bare_subscript():
    bad = []
    for src in sorted(CSRC.glob("*.h")) + sorted(CSRC.glob("*.hip")):
        text = re.sub(r"\s+", " ", src.read_text())
        bad += [f"{src.name}: {m.group(0)}" for m in BARE_SUBSCRIPT.finditer(text)]
    assert not bad, bad


PROBE = """
#include <hip/hip_runtime.h>
#include <stdint.h>
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__global__ void k_probe(float* dst, const u32x4* src) {
    const u32x4 v = src[threadIdx.x];
#pragma unroll
    for (int j = 0; j < 4; ++j) dst[j * 64 + threadIdx.x] = __builtin_bit_cast(float, (uint32_t)v[j]);
}
"""


def test_rvalue_bit_cast_reads_every_vector_element(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc is not installed")
    src = tmp_path / "probe.hip"
    src.write_text(PROBE)
    asm = tmp_path / "probe.s"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "--cuda-device-only", "-S", str(src), "-o", str(asm)],
                   check=True, capture_output=True)
    stores = re.findall(r"global_store_dword \S+, (v\d+),", asm.read_text())
    assert len(stores) == 4 and len(set(stores)) == 4, stores
