"""Builds the MI355X backend libraries in-tree.

Outputs (git-ignored, shipped with the tree to the GPU host):
  mlvc.cpp_amd/lib/libmlvc_hip_device.so  gfx950 kernels + device C ABI (hipcc)
  mlvc.cpp_amd/lib/libmlvc_hip.so         C++20 runtime + "hip" backend + backend C ABI (g++); with
                                          MLVC_EMBED_MODEL_ROOT=<dir>, also the model bundles below <dir>
                                          (<profile>/<WxH>/) as an embedded image (python/mlvc_embed.py;
                                          MLVC_EMBED_PROFILES=<profiles.json> selects and orders them)
  oracle/liboracle.so                     CPU oracle (test infrastructure, g++)
  oracle/_ref/libmlvc_ref_kernels.so      reference CPU kernels, when the reference checkout exists

Run `python mlvc.cpp_amd/build.py` or call build_all().
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
REPO = PKG.parent
LIB = PKG / "lib"
OBJ = PKG / "_build"
ORACLE = REPO / "oracle"
ROCM = pathlib.Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = os.environ.get("MLVC_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC",
    # Packed FP32 instructions stay disabled for all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO / 'include'}", f"-I{PKG / 'csrc'}",
]
CXX_FLAGS = ["-std=c++20", "-O2", "-fPIC", "-Wall", "-Wextra",
             f"-I{PKG / 'runtime' / 'include'}", f"-I{REPO / 'include'}"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")


def _objects(sources, compiler, flags, jobs):
    OBJ.mkdir(parents=True, exist_ok=True)
    objs, cmds = [], []
    for src in sources:
        obj = OBJ / (src.parent.name + "_" + src.name + ".o")
        objs.append(str(obj))
        cmds.append([compiler, *flags, "-c", str(src), "-o", str(obj)])
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        for fut in [pool.submit(_run, c) for c in cmds]:
            fut.result()
    return objs


def build_all(jobs: int | None = None, verbose: bool = True) -> None:
    jobs = jobs or min(8, os.cpu_count() or 4)
    LIB.mkdir(parents=True, exist_ok=True)
    hip_srcs = sorted((PKG / "csrc").glob("*.hip"))
    cpp_srcs = sorted((PKG / "runtime" / "src").glob("*.cpp")) + sorted((PKG / "backend_hip" / "src").glob("*.cpp"))
    with concurrent.futures.ThreadPoolExecutor(max_workers=3) as pool:
        dev = pool.submit(_objects, hip_srcs, HIPCC, HIP_FLAGS, jobs)
        host = pool.submit(_objects, cpp_srcs, "g++", CXX_FLAGS, jobs)
        orc = pool.submit(_run, ["g++", "-std=c++20", "-O3", "-fPIC", "-shared", "-mavx2", "-mfma", "-mf16c",
                                 "-ffp-contract=off", str(ORACLE / "cpu_oracle.cpp"), "-o",
                                 str(ORACLE / "liboracle.so"), "-lpthread"])
        dev_objs, host_objs = dev.result(), host.result()
        orc.result()
    dev_lib = LIB / "libmlvc_hip_device.so"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *dev_objs, "-o", str(dev_lib)])
    link_host = ["g++", "-shared", *host_objs, f"-L{LIB}", "-lmlvc_hip_device", "-Wl,-rpath,$ORIGIN",
                 "-o", str(LIB / "libmlvc_hip.so"), "-lpthread"]
    _run(link_host)
    embed_root = os.environ.get("MLVC_EMBED_MODEL_ROOT")
    if embed_root:
        # Embedded model image: the packer checks every bundle through the
        # library just linked, then the library is linked again with the
        # image's objects (the payload is .incbin'd at assembly time).
        out = OBJ / "embedded-models"
        registry = os.environ.get("MLVC_EMBED_PROFILES")
        _run([sys.executable, str(PKG / "python" / "mlvc_embed.py"), "--model-root", embed_root, "--out-dir", str(out)]
             + (["--profiles", registry] if registry else []))
        image = []
        for src in ("mlvc_embedded_models.S", "mlvc_embedded_models_index.c"):
            image.append(str(out / (src + ".o")))
            _run(["gcc", "-c", "-fPIC", f"-I{REPO / 'include'}", str(out / src), "-o", image[-1]])
        _run(link_host[:-3] + image + link_host[-3:])
    ref_script = ORACLE / "build_ref.sh"
    if pathlib.Path("/root/reference/backends/cpu/src").is_dir():
        _run(["bash", str(ref_script)])
    shutil.rmtree(OBJ, ignore_errors=True)
    if verbose:
        print(f"built {dev_lib}, {LIB / 'libmlvc_hip.so'}, {ORACLE / 'liboracle.so'}")


if __name__ == "__main__":
    build_all()
    sys.exit(0)
