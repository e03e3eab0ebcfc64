"""Builds the in-tree shared libraries of voxgen_amd.

  voxgen_amd/libvoxhip.so    HIP kernels for gfx950 + C ABI (include/voxhip.h)
  voxgen_amd/libvoxsynth.so  host-side deterministic input generator

`--timeline` instead builds voxgen_amd/timeline/libvoxhip.so with -DVX_STAMPS: the
same library whose decode kernels also record per-wave s_memrealtime ticks
(vx_diag_timeline_*), loaded through VOXHIP_LIBRARY by `bench.py --timeline`.

Device code is compiled with packed-FP32 instructions disabled
(-Xclang -target-feature -Xclang -packed-fp32-ops).
Run as a script or call build_all(); every call recompiles.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
ROOT = PKG.parent
OBJ = ROOT / "_build" / "voxhip"
ARCH = os.environ.get("VOXHIP_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
HIP_FLAGS = [
    "-x", "hip", f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError("command failed:\n" + " ".join(cmd) + "\n" + proc.stdout)
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "packed-fp32-ops" not in l and l.strip())
    if out.strip():
        print(out, file=sys.stderr)


# Per-file device flags. The prefill GEMM keeps its MFMA accumulators in
# VGPRs: its per-block scale FMAs read them, and accumulators in AGPRs would cost
# a v_accvgpr_read per element.
FILE_FLAGS = {
    "kernels_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


# Host-side AddressSanitizer + UndefinedBehaviorSanitizer build, for the CPU
# tests of the host code (GGUF parsing, argument checks). Each sanitizer flag is
# scoped to the host pass with -Xarch_host; the device code is built as usual.
SANITIZE_HOST = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                 "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer",
                 "-Xarch_host", "-shared-libasan"]
ASAN_DIR = ROOT / "_build" / "asan"
TIMELINE_OBJ = ROOT / "_build" / "timeline"
TIMELINE_DIR = PKG / "timeline"


def _compile(src: Path, sanitize: bool = False, timeline: bool = False) -> Path:
    odir = ASAN_DIR / "obj" if sanitize else TIMELINE_OBJ if timeline else OBJ
    odir.mkdir(parents=True, exist_ok=True)
    obj = odir / (src.name + ".o")
    # hipcc treats .cpp as HIP source too; both get the gfx950 device flags.
    cmd = [HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(src.name, []), *(SANITIZE_HOST if sanitize else []),
           *(["-DVX_STAMPS"] if timeline else []), "-c", str(src), "-o", str(obj)]
    _run(cmd)
    return obj


def build_voxhip(jobs: int | None = None, sanitize: bool = False, timeline: bool = False) -> Path:
    """Build libvoxhip.so in the package; with sanitize=True the host-sanitized
    variant at _build/asan/libvoxhip.so (load it with VOXHIP_LIBRARY and the ASan
    runtime preloaded); with timeline=True the -DVX_STAMPS variant at
    voxgen_amd/timeline/libvoxhip.so."""
    sources = sorted(CSRC.glob("*.hip")) + sorted(
        p for p in CSRC.glob("*.cpp"))
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda src: _compile(src, sanitize, timeline), sources))
    out = (ASAN_DIR if sanitize else TIMELINE_DIR if timeline else PKG) / "libvoxhip.so"
    out.parent.mkdir(parents=True, exist_ok=True)
    tmp = out.with_name("libvoxhip.so.tmp")
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *(SANITIZE_HOST if sanitize else []),
          "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, out)
    return out


def asan_runtime() -> str:
    """Path of the clang ASan runtime that a sanitized build needs preloaded."""
    clang = Path(HIPCC).resolve().parent.parent / "lib" / "llvm" / "bin" / "clang"
    if not clang.exists():
        clang = Path(shutil.which("clang") or "/opt/rocm/lib/llvm/bin/clang")
    return subprocess.run([str(clang), "-print-file-name=libclang_rt.asan-x86_64.so"], check=True,
                          stdout=subprocess.PIPE, text=True).stdout.strip()


def build_synth() -> Path:
    out = PKG / "libvoxsynth.so"
    tmp = PKG / "libvoxsynth.so.tmp"
    _run(["gcc", "-O3", "-march=x86-64-v3", "-fopenmp", "-fPIC", "-shared", "-std=c11",
          "-Wall", "-o", str(tmp), str(CSRC / "synth.c"), "-lm"])
    os.replace(tmp, out)
    return out


def build_all(verbose: bool = False) -> None:
    with cf.ThreadPoolExecutor(max_workers=1) as ex:
        f_syn = ex.submit(build_synth)
        hip = build_voxhip()
        syn = f_syn.result()
    if verbose:
        for p in (hip, syn):
            print(f"built {p.relative_to(ROOT)}")


if __name__ == "__main__":
    if "--timeline" in sys.argv[1:]:
        print(f"built {build_voxhip(timeline=True).relative_to(ROOT)}")
    else:
        build_all(verbose=True)
