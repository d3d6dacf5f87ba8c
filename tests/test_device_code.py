"""The gfx950 code in the built device library holds no instruction that
would change the rounding the kernels promise (disassembled here, no GPU).

* v_fma_mix{lo,hi}_f16 / v_mad_mix{lo,hi}_f16 round an FP32 multiply-add
  straight to FP16 once. The kernels round like the reference CPU kernels:
  the FP32 result first, then to FP16. The compiler forms these from
  f2h(fmaf(...)) unless the value is kept opaque, and the difference shows
  only on rare inputs, so it is checked on the code itself.
* Packed FP32 arithmetic (v_pk_fma_f32, v_pk_mul_f32, v_pk_add_f32) is
  disabled for all device code by the build flags; none may appear.

The library's .hip_fatbin section is a sequence of offload bundles (one per
HIP source); each one's gfx950 code object is unbundled and disassembled.
"""

import pathlib
import re
import subprocess

import pytest

import mlvc_hip

LLVM = pathlib.Path("/opt/rocm/llvm/bin")
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
FORBIDDEN = re.compile(r"\b(v_(?:fma|mad)_mix(?:lo|hi)_f16|v_pk_(?:fma|mul|add)_f32)\b")

pytestmark = pytest.mark.skipif(not (LLVM / "llvm-objdump").exists(), reason="ROCm LLVM tools not available")


@pytest.fixture(scope="module")
def disassembly(tmp_path_factory):
    out = tmp_path_factory.mktemp("isa")
    fatbin = out / "fatbin.bin"
    subprocess.run(["objcopy", f"--dump-section=.hip_fatbin={fatbin}", str(mlvc_hip.DEVICE_LIB), str(out / "lib.so")],
                   check=True, capture_output=True)
    data = fatbin.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
    assert starts, "no offload bundle in the device library"
    texts = []
    for k, st in enumerate(starts):
        end = starts[k + 1] if k + 1 < len(starts) else len(data)
        b, co = out / f"b{k}.bin", out / f"c{k}.o"
        b.write_bytes(data[st:end])
        subprocess.run([str(LLVM / "clang-offload-bundler"), "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                        f"--input={b}", f"--output={co}", "--unbundle"], check=True, capture_output=True)
        texts.append(subprocess.run([str(LLVM / "llvm-objdump"), "-d", str(co)], check=True, capture_output=True,
                                    text=True).stdout)
    return texts


def test_device_library_holds_gfx950_kernels(disassembly):
    assert sum(t.count("v_mfma") for t in disassembly) > 1000  # the conv kernels
    assert all("elf64-amdgpu" in t for t in disassembly)


def test_no_single_rounding_mix_or_packed_fp32(disassembly):
    bad = set()
    for text in disassembly:
        kernel = None
        for line in text.splitlines():
            if line.endswith(">:"):
                kernel = line.split("<", 1)[-1][:-2]
            m = FORBIDDEN.search(line)
            if m:
                bad.add((kernel, m.group(1)))
    assert not bad, sorted(bad)[:20]
