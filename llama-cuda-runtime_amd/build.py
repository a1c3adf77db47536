"""Builds the HIP shared libraries of the token loop for gfx950.

Two variants, as the reference's LCR_DTYPE switch gives two builds
(CMakeLists.txt:79-99):
  liblcr_amd.so       bf16 elements (default)
  liblcr_amd_fp16.so  fp16 elements (-DLCR_ELEM_FP16)

The command-line programs of csrc/tools/ (llama-run, lcr-validate,
lcr-inspect) are linked against those libraries into bin/.

Every source is compiled with hipcc for gfx950 only, with -ffp-contract=off so
that only the explicit fma calls in the kernels are fused (the kernels'
summation orders are part of their contract), and with packed fp32 operations
disabled. Objects go to _build/<variant>/, libraries next to this file.

Usage: python build.py [--jobs N] [--variant bf16|fp16|all]
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON_FLAGS = [
    "-std=c++17",
    "-O3",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
    f"-I{REPO / 'include'}",
    f"-I{CSRC}",
]

VARIANTS = {
    "bf16": ("liblcr_amd.so", []),
    "fp16": ("liblcr_amd_fp16.so", ["-DLCR_ELEM_FP16"]),
}


def sources() -> list[Path]:
    out = sorted(CSRC.glob("*.cpp")) + sorted((CSRC / "kernels").glob("*.hip"))
    return out


def _compile(src: Path, obj: Path, defines: list[str]) -> tuple[Path, int, str]:
    obj.parent.mkdir(parents=True, exist_ok=True)
    lang = ["-x", "hip"] if src.suffix == ".hip" else ["-x", "hip"]
    cmd = [HIPCC, *COMMON_FLAGS, *defines, *lang, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    text = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines()
        if "packed-fp32-ops" not in line
    )
    return src, proc.returncode, text


def build_variant(name: str, jobs: int) -> Path:
    lib_name, defines = VARIANTS[name]
    objdir = PKG / "_build" / name
    srcs = sources()
    objs = []
    failures = []
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        futs = []
        for src in srcs:
            rel = src.relative_to(CSRC)
            obj = objdir / (str(rel).replace("/", "__") + ".o")
            objs.append(obj)
            futs.append(pool.submit(_compile, src, obj, defines))
        for fut in futs:
            src, rc, text = fut.result()
            if text.strip():
                print(f"[{name}] {src.name}:\n{text}", file=sys.stderr)
            if rc != 0:
                failures.append(src.name)
    if failures:
        raise RuntimeError(f"{name}: compilation failed for {', '.join(failures)}")
    lib = PKG / lib_name
    tmp = lib.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *[str(o) for o in objs], "-lpthread"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"{name}: link failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, lib)
    return lib


# Command-line programs (csrc/tools/<name>_main.cpp), linked against the bf16
# library (the fp16 build when its name ends in -fp16), into bin/.
TOOLS = {
    "llama-run": ("run_main.cpp", "bf16"),
    "llama-run-fp16": ("run_main.cpp", "fp16"),
    "lcr-validate": ("validate_main.cpp", "bf16"),
    "lcr-inspect": ("inspect_main.cpp", "bf16"),
}


def _build_tool(name: str, source: str, variant: str) -> tuple[str, int, str]:
    lib_name, defines = VARIANTS[variant]
    out = PKG / "bin" / name
    out.parent.mkdir(exist_ok=True)
    tmp = out.with_name(out.name + ".tmp")
    cmd = [HIPCC, *COMMON_FLAGS, *defines, "-x", "hip", str(CSRC / "tools" / source), "-o", str(tmp),
           f"-L{PKG}", f"-l:{lib_name}", "-Wl,-rpath,$ORIGIN/.."]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    text = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines() if "packed-fp32-ops" not in line)
    if proc.returncode == 0:
        os.replace(tmp, out)
    return name, proc.returncode, text


def build_tools(variants: list[str], jobs: int) -> list[Path]:
    todo = [(n, s, v) for n, (s, v) in TOOLS.items() if v in variants]
    failures = []
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        for name, rc, text in pool.map(lambda t: _build_tool(*t), todo):
            if text.strip():
                print(f"[{name}]:\n{text}", file=sys.stderr)
            if rc != 0:
                failures.append(name)
    if failures:
        raise RuntimeError(f"tools failed to build: {', '.join(failures)}")
    return [PKG / "bin" / n for n, _, _ in todo]


def build(variants: list[str] | None = None, jobs: int | None = None) -> list[Path]:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    jobs = jobs or min(16, os.cpu_count() or 4)
    variants = variants or list(VARIANTS)
    libs = [build_variant(v, jobs) for v in variants]
    return libs + build_tools(variants, jobs)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--variant", default="all", choices=["all", *VARIANTS])
    args = ap.parse_args()
    variants = list(VARIANTS) if args.variant == "all" else [args.variant]
    for lib in build(variants, args.jobs):
        print(f"built {lib}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
