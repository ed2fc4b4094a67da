"""Build the HIP C-ABI library ``mogt_amd/lib/libmogt_hip.so`` for gfx950.

The library is plain HIP (no torch headers): every ``csrc/*.hip`` file is
compiled with ``hipcc --offload-arch=gfx950`` and linked into one shared object
that Python loads through ctypes (``mogt_amd._lib``).  The build is in-tree so
the ``.so`` travels with the source tree to the GPU host.
"""
from __future__ import annotations

import concurrent.futures as cf
import hashlib
import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
LIBNAME = "libmogt_hip.so"
INCLUDE = PKG.parent / "include"

ARCH = os.environ.get("MOGT_OFFLOAD_ARCH", "gfx950")

# Packed-FP32 VALU forms are switched off for every device compile.
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-rdc",
    "-Wall",
    "-Wno-unused-function",
]

# Per-file extras.  The rank-1 kernels rescale MFMA accumulators between
# chains; keeping accumulators in ordinary VGPRs avoids a copy to and from the
# accumulation registers around every such rescale.
FILE_FLAGS = {
    "rank1_scan.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def source_manifest() -> dict[str, str]:
    """Build identity: ``name -> sha256[:12]`` of every source the library is
    compiled from (``csrc/*.hip``, ``csrc/*.h``, the public header) plus the
    compiler flags (key ``flags``).  The same string is compiled into the
    library (``mogt_build_manifest``), so a loaded library can be matched
    against the tree, and a profile taken from one build can name the exact
    sources its kernels came from."""
    files = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.h")) + [INCLUDE / "mogt_scan.h"]
    out = {f.name: hashlib.sha256(f.read_bytes()).hexdigest()[:12] for f in files}
    flags = repr((HIPCC_FLAGS, sorted(FILE_FLAGS.items())))
    out["flags"] = hashlib.sha256(flags.encode()).hexdigest()[:12]
    return out


def manifest_string(manifest: dict[str, str]) -> str:
    return ";".join(f"{k}:{v}" for k, v in sorted(manifest.items()))


def parse_manifest(text: str) -> dict[str, str]:
    return dict(item.split(":", 1) for item in text.split(";") if ":" in item)


def build_id(manifest: dict[str, str]) -> str:
    """Short hash of a whole manifest (one id per library build)."""
    return hashlib.sha256(manifest_string(manifest).encode()).hexdigest()[:16]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: the MOGT HIP library cannot be built")
    return exe


def lib_path() -> Path:
    return LIBDIR / LIBNAME


def _compile(src: Path, obj: Path, defines: tuple[str, ...] = ()) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, []), *defines, f"-I{INCLUDE}", "-c", str(src),
           "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    # hipcc's host pass does not know the packed-fp32 feature (harmless).  The
    # bf16 GEMMs set m0 in inline assembly for their direct-to-LDS loads
    # (lds_dma.h), which clang flags as a reserved register on a clobber list;
    # that m0 is
    # written only there and read only by the load that follows is checked on
    # the generated code by tests/test_host_logic.py, so the warning is counted
    # here rather than repeated per inlined call.
    lines = res.stderr.splitlines()
    m0 = sum("clobber list contains reserved registers: m0" in ln for ln in lines)
    noise = [ln for ln in lines
             if ln.strip() and "packed-fp32-ops" not in ln
             and "clobber list contains reserved registers: m0" not in ln
             and "Reserved registers on the clobber list" not in ln
             and not (m0 and ("lds_dma16" in ln or "s_mov_b32 m0" in ln or ln.strip().startswith(("|", "^"))
                              or ln.strip()[:1].isdigit() or "in asm" in ln or "note:" in ln
                              or (ln.startswith("In file included from") and "lds_dma.h" not in ln)))
             and not ln.strip().endswith("warnings generated.") and not ln.strip().endswith("warning generated.")]
    if m0:
        print(f"[mogt build] {src.name}: {m0} inline-asm m0 clobber warnings (direct-to-LDS loads; "
              "m0 use checked by tests/test_host_logic.py)")
    if noise:
        print(f"[mogt build] {src.name}:\n" + "\n".join(noise))


def build(verbose: bool = True, jobs: int | None = None) -> Path:
    """Compile every ``csrc/*.hip`` and link ``lib/libmogt_hip.so``."""
    LIBDIR.mkdir(parents=True, exist_ok=True)
    objdir = LIBDIR / "obj"
    objdir.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [objdir / (s.stem + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), max(1, os.cpu_count() or 2))
    manifest = manifest_string(source_manifest())
    defines = [(f'-DMOGT_BUILD_MANIFEST="{manifest}"',) if s.name == "capi.hip" else () for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_compile, srcs, objs, defines))
    out = lib_path()
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    for o in objs:
        o.unlink(missing_ok=True)
    if verbose:
        print(f"[mogt build] wrote {out}")
    return out


if __name__ == "__main__":
    build()
