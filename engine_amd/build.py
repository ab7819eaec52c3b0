"""Builds engine_amd/libribn_amd.so (HIP kernels + C ABI) for gfx950 with hipcc.

    python -m engine_amd.build                      # the product library
    python -m engine_amd.build --sanitize           # host code under ASan + UBSan
    python -m engine_amd.build --resource-report F  # per-kernel registers, LDS, scratch

Compiles every translation unit under engine_amd/csrc in parallel and links one
shared library in-tree, next to this file, so it travels with the repository.

`--sanitize` builds engine_amd/_build_asan/libribn_amd_asan.so: the same
sources with AddressSanitizer and UndefinedBehaviorSanitizer on the host side
only (every flag behind -Xarch_host; device code is compiled exactly as in the
product). It is a CPU test artefact: a process loads it with
RIBN_AMD_LIBRARY=<path> and the clang ASan runtime preloaded
(tests/test_sanitizers.py does both).

`--resource-report F` compiles with the compiler's kernel-resource-usage
remarks and writes F, a table of every instantiated kernel: SGPRs, VGPRs,
AGPRs, scratch bytes per lane (spills), LDS bytes and occupancy in waves per
SIMD. It prints the same kind of per-kernel attributes the reference logs at
load time under RIBN_LOG_KERNEL_ATTRS (crates/nvidia/src/quantized.rs:224-237),
taken here at compile time because gfx950 code objects are built ahead.
"""
from __future__ import annotations

import argparse
import concurrent.futures
import os
import re
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libribn_amd.so")
ASAN_OBJ = os.path.join(HERE, "_build_asan")
ASAN_LIB = os.path.join(ASAN_OBJ, "libribn_amd_asan.so")
ARCH = os.environ.get("RIBN_AMD_ARCH", "gfx950")

# Packed-FP32 instructions are disabled for all device code on this platform.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Products and sums round separately unless a kernel asks for an FMA
    # (__builtin_fmaf): keeps the exact-order kernels bit-identical to the host.
    "-ffp-contract=off",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
    "-Wall", "-Wno-unused-function",
]

# Host-only sanitizers: hipcc applies each flag after -Xarch_host to the host
# compilation alone.
SANITIZE_FLAGS = [
    "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer",
]
SANITIZE_LINK = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                 "-Xarch_host", "-shared-libsan"]

SOURCES = ["kquant_kernels.hip", "gemv_wave.hip", "gemv_f32.hip", "gemv_mfma.hip", "gemv_f32mma.hip", "q8_1.hip", "qgemm.hip", "decode_kernels.hip", "probe.hip", "ribn_amd.cpp", "qwen3_decode.cpp", "gguf.cpp", "serving.cpp"]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; ROCm is required to build engine_amd")
    return path


def _compile(src: str, obj_dir: str = OBJ, extra: tuple = ()) -> tuple[str, str]:
    obj = os.path.join(obj_dir, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj, res.stderr


def _link(objs: list[str], out: str, extra: tuple = ()) -> None:
    tmp = out + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, *extra]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)


def _compile_all(obj_dir: str, extra: tuple = ()) -> list[tuple[str, str]]:
    os.makedirs(obj_dir, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        return list(pool.map(lambda src: _compile(src, obj_dir, extra), SOURCES))


def build(verbose: bool = False) -> str:
    """Builds the product library; returns its path."""
    objs = [o for o, _ in _compile_all(OBJ)]
    _link(objs, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def build_sanitized(verbose: bool = False) -> str:
    """Builds the host-sanitized test library; returns its path."""
    objs = [o for o, _ in _compile_all(ASAN_OBJ, tuple(SANITIZE_FLAGS))]
    _link(objs, ASAN_LIB, tuple(SANITIZE_LINK))
    if verbose:
        print(f"built {ASAN_LIB}")
    return ASAN_LIB


def sanitized_is_current() -> bool:
    """True when the sanitized library is newer than every source and header."""
    if not os.path.exists(ASAN_LIB):
        return False
    built = os.path.getmtime(ASAN_LIB)
    for d in (CSRC, os.path.join(ROOT, "include")):
        for name in os.listdir(d):
            if os.path.getmtime(os.path.join(d, name)) > built:
                return False
    return True


_REMARK = re.compile(r"(?P<src>[^\s:]+):\d+:\d+: remark: (?P<key>[^:]+?): (?P<val>.*)$")
_FIELDS = {"TotalSGPRs": "sgpr", "VGPRs": "vgpr", "AGPRs": "agpr", "ScratchSize [bytes/lane]": "scratch",
           "SGPRs Spill": "sgpr_spill", "VGPRs Spill": "vgpr_spill", "Occupancy [waves/SIMD]": "occupancy",
           "LDS Size [bytes/block]": "lds"}


def parse_resource_remarks(text: str) -> list[dict]:
    """Kernels and their resources from -Rpass-analysis=kernel-resource-usage output."""
    kernels, cur = [], None
    for line in text.splitlines():
        m = _REMARK.search(line)
        if not m:
            continue
        key = m.group("key").strip()
        val = re.sub(r"\s*\[-R[^\]]*\]$", "", m.group("val")).strip()
        if key == "Function Name":
            cur = {"source": os.path.basename(m.group("src")), "kernel": val}
            kernels.append(cur)
        elif cur is not None and key in _FIELDS:
            cur[_FIELDS[key]] = int(val)
    return kernels


def resource_report(path: str, verbose: bool = False) -> list[dict]:
    """Compiles every source with kernel-resource-usage remarks into a scratch
    object directory and writes a markdown table of every kernel to `path`."""
    flags = ("-Rpass-analysis=kernel-resource-usage",)
    results = _compile_all(os.path.join(OBJ, "resource_report"), flags)
    kernels = []
    for _, err in results:
        kernels += parse_resource_remarks(err)
    demangled = _demangle([k["kernel"] for k in kernels])
    lines = [
        "# Kernel resources (gfx950)",
        "",
        "Compiler resource-usage remarks for every kernel in libribn_amd.so, one row",
        "per instantiation: scalar, vector and accumulation registers, scratch bytes",
        "per lane (register spills or stack arrays), spilled SGPRs and VGPRs, LDS",
        "bytes per workgroup, and the occupancy bound in waves per SIMD.",
        "",
        "Command: `python -m engine_amd.build --resource-report profiles/kernel_resources.md`",
        f"(flags: {' '.join(_code_flags())} -Rpass-analysis=kernel-resource-usage).",
        "",
        "| source | kernel | SGPR | VGPR | AGPR | scratch B/lane | SGPR spill | VGPR spill | LDS B | waves/SIMD |",
        "|---|---|---:|---:|---:|---:|---:|---:|---:|---:|",
    ]
    for k, name in sorted(zip(kernels, demangled), key=lambda kn: (kn[0]["source"], kn[1])):
        lines.append(f"| {k['source']} | `{name}` | {k.get('sgpr', '')} | {k.get('vgpr', '')} | "
                     f"{k.get('agpr', '')} | {k.get('scratch', '')} | {k.get('sgpr_spill', '')} | "
                     f"{k.get('vgpr_spill', '')} | {k.get('lds', '')} | "
                     f"{k.get('occupancy', '')} |")
    scratch = [n for k, n in zip(kernels, demangled) if k.get("scratch", 0) > 0]
    spills = [n for k, n in zip(kernels, demangled) if k.get("vgpr_spill", 0) + k.get("sgpr_spill", 0) > 0]
    lines += ["", f"{len(kernels)} kernels; {len(scratch)} use scratch"
              + (": " + ", ".join(f"`{n}`" for n in scratch) if scratch else "")
              + f"; {len(spills)} spill registers"
              + (": " + ", ".join(f"`{n}`" for n in spills) if spills else "") + "."]
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")
    if verbose:
        print(f"wrote {path}: {len(kernels)} kernels")
    return kernels


def _code_flags() -> list[str]:
    """HIPCC_FLAGS without include paths and warning switches."""
    out, skip = [], False
    for f in HIPCC_FLAGS:
        if skip:
            skip = False
        elif f == "-I":
            skip = True
        elif not f.startswith("-W"):
            out.append(f)
    return out


def _short_name(name: str) -> str:
    """A demangled kernel name without namespaces, return type and parameter list."""
    name = name.replace("(anonymous namespace)::", "").replace("ribn_amd::", "")
    if name.startswith("void "):
        name = name[5:]
    depth = 0
    for i, c in enumerate(name):
        depth += c == "<"
        depth -= c == ">"
        if c == "(" and depth == 0:
            return name[:i]
    return name


def _demangle(names: list[str]) -> list[str]:
    """c++filt where it knows the mangling; names it leaves mangled (binutils
    does not know `DF16_`, the _Float16 parameter code) go through the kernel
    name reader of engine_amd.profiling, which keeps the template arguments."""
    from engine_amd.profiling import short_name

    tool = shutil.which("c++filt") or shutil.which("llvm-cxxfilt")
    out = names
    if names and tool:
        res = subprocess.run([tool], input="\n".join(names), capture_output=True, text=True)
        lines = res.stdout.splitlines()
        if res.returncode == 0 and len(lines) == len(names):
            out = lines
    return [short_name(n) if n.startswith("_Z") else _short_name(n) for n in out]


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--sanitize", action="store_true", help="build the host-sanitized test library")
    ap.add_argument("--resource-report", metavar="PATH", help="write the per-kernel resource table to PATH")
    a = ap.parse_args()
    if a.resource_report:
        resource_report(a.resource_report, verbose=True)
    elif a.sanitize:
        build_sanitized(verbose=True)
    else:
        build(verbose=True)
    sys.exit(0)
