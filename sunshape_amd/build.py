"""Builds the sunshape_amd HIP library (gfx950) and its torch operators in-tree.

``python -m sunshape_amd.build`` or ``sunshape_amd.build.build()`` compiles every
``csrc/*.hip`` source into ``sunshape_amd/_lib/libsunshape_amd.so`` (each source to an object in
``sunshape_amd/_lib/obj``, in parallel, then linked) and ``csrc/torch_ops.cpp`` into
``sunshape_amd/_lib/libsunshape_torch_ops.so`` (torch.ops.sunshape.*).  ``csrc/probe/*.hip`` (a
bandwidth probe bench.py times beside the decode) links separately into
``sunshape_amd/_lib/libsunshape_probe.so``.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_lib")
LIB_PATH = os.path.join(OUT_DIR, "libsunshape_amd.so")
TORCH_OPS_PATH = os.path.join(OUT_DIR, "libsunshape_torch_ops.so")
PROBE_PATH = os.path.join(OUT_DIR, "libsunshape_probe.so")  # measurement probes (bench.py), not the library
ARCH = "gfx950"

# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 in generated code.
# -ffp-contract=off: every multiply-add the sources want fused is an explicit fmaf; the
# encode kernels reproduce a reference rounding sequence bit-for-bit.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the sunshape_amd HIP library cannot be built")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _build_torch_ops() -> None:
    """torch.ops.sunshape.* (csrc/torch_ops.cpp): host C++ against torch's headers, linked to the
    HIP library (found next to it through $ORIGIN) and to torch's libraries."""
    import torch.utils.cpp_extension as ext

    import torch

    src = os.path.join(CSRC, "torch_ops.cpp")
    tlib = ext.library_paths()[0]
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           *[f"-I{p}" for p in ext.include_paths()], "-I/opt/rocm/include", src,
           "-o", TORCH_OPS_PATH + ".tmp", f"-L{OUT_DIR}", "-lsunshape_amd", f"-L{tlib}", "-lc10", "-lc10_hip",
           "-ltorch_cpu", "-ltorch", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{tlib}"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"torch operators failed to build:\n{res.stderr}")
    os.replace(TORCH_OPS_PATH + ".tmp", TORCH_OPS_PATH)


def _compile(hipcc: str, src: str, obj: str) -> None:
    cmd = [hipcc, *HIP_FLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (res.stderr or "").splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {os.path.basename(src)}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def _includes(path: str, seen: set) -> None:
    """Local headers path includes (#include "..."), recursively, into seen."""
    for line in open(path):
        line = line.strip()
        if line.startswith("#include") and '"' in line:
            dep = os.path.normpath(os.path.join(os.path.dirname(path), line.split('"')[1]))
            if os.path.exists(dep) and dep not in seen:
                seen.add(dep)
                _includes(dep, seen)


def _stale(src: str, obj: str) -> bool:
    if not os.path.exists(obj):
        return True
    deps = {src}
    _includes(src, deps)
    t = os.path.getmtime(obj)
    return any(t < os.path.getmtime(d) for d in deps)


def build(verbose: bool = False, incremental: bool = False) -> str:
    """Compile all HIP sources and link the shared library; returns its path.

    incremental: recompile only sources whose object is older than the source or than a header
    it includes (a development shortcut; the default rebuilds everything).
    """
    hipcc = _hipcc()
    obj_dir = os.path.join(OUT_DIR, "obj")
    os.makedirs(obj_dir, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(obj_dir, os.path.basename(s)[:-4] + ".o") for s in srcs]
    work = list(zip(srcs, objs))
    if incremental:
        work = [(s, o) for s, o in work if _stale(s, o)]
        if verbose:
            print("compiling:", " ".join(os.path.basename(s) for s, _ in work) or "(nothing)")
    if work:
        with cf.ThreadPoolExecutor(max_workers=min(8, len(work))) as ex:
            list(ex.map(lambda so: _compile(hipcc, *so), work))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if not incremental or not os.path.exists(TORCH_OPS_PATH) or \
            os.path.getmtime(TORCH_OPS_PATH) < max(os.path.getmtime(os.path.join(CSRC, "torch_ops.cpp")),
                                                   os.path.getmtime(os.path.join(os.path.dirname(HERE), "include",
                                                                                 "sunshape_amd.h"))):
        _build_torch_ops()
    probe_src = os.path.join(CSRC, "probe", "ssq_probe_stream.hip")
    if not incremental or not os.path.exists(PROBE_PATH) or os.path.getmtime(PROBE_PATH) < os.path.getmtime(probe_src):
        cmd = [hipcc, *HIP_FLAGS, "-shared", probe_src, "-o", PROBE_PATH + ".tmp"]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"probe library failed to build:\n{res.stderr}")
        os.replace(PROBE_PATH + ".tmp", PROBE_PATH)
    if verbose:
        print(f"built {LIB_PATH}, {TORCH_OPS_PATH} and {PROBE_PATH}")
    return LIB_PATH


SAN_DIR = os.path.join(OUT_DIR, "san")
SAN_LIB_PATH = os.path.join(SAN_DIR, "libsunshape_amd_hostsan.so")


def asan_runtime() -> str | None:
    """The compiler's shared AddressSanitizer runtime (to LD_PRELOAD into a process that loads the
    host-sanitized library), or None."""
    import glob

    hits = sorted(glob.glob("/opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return hits[-1] if hits else None


def build_host_sanitized(verbose: bool = False) -> str:
    """The library with its host code under AddressSanitizer and UndefinedBehaviorSanitizer (each
    -fsanitize= behind -Xarch_host: the device code is built plainly, at -O1, since a host-only
    object would reference a fatbin nothing defines), for CPU tests that drive the argument checks
    and launch planning with arbitrary inputs in a process that sees no GPU.  Rebuilt when a source
    or header is newer than the library.  Returns the library's path."""
    hipcc = _hipcc()
    os.makedirs(SAN_DIR, exist_ok=True)
    srcs = sources()
    if os.path.exists(SAN_LIB_PATH):
        t = os.path.getmtime(SAN_LIB_PATH)
        deps = set(srcs)
        for s in srcs:
            _includes(s, deps)
        if all(os.path.getmtime(d) <= t for d in deps):
            return SAN_LIB_PATH
    san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer"]
    flags = [f"--offload-arch={ARCH}", "-O1", "-Xarch_host", "-g", "-std=c++17", "-fPIC", "-ffp-contract=off",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", *san]
    objs = [os.path.join(SAN_DIR, os.path.basename(s)[:-4] + ".o") for s in srcs]

    def one(so):
        src, obj = so
        res = subprocess.run([hipcc, *flags, "-c", src, "-o", obj], capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"host-sanitized compile failed for {os.path.basename(src)}:\n{res.stderr}")

    with cf.ThreadPoolExecutor(max_workers=8) as ex:
        list(ex.map(one, zip(srcs, objs)))
    tmp = SAN_LIB_PATH + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-shared-libsan", "-Xarch_host", "-fsanitize=address",
           "-Xarch_host", "-fsanitize=undefined", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"host-sanitized link failed:\n{res.stderr}")
    os.replace(tmp, SAN_LIB_PATH)
    if verbose:
        print(f"built {SAN_LIB_PATH}")
    return SAN_LIB_PATH


if __name__ == "__main__":
    if "--host-sanitized" in sys.argv[1:]:
        build_host_sanitized(verbose=True)
    else:
        build(verbose=True, incremental="--incremental" in sys.argv[1:])
