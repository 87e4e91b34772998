"""Build recipe of the in-tree HIP library ``_build/libloom_hip.so`` (gfx950).

hipcc compiles the paged-decode kernels with the C ABI and the RoPE + paged
K/V write kernel into one shared library. Packed FP32 instruction selection is
disabled (``-packed-fp32-ops``) for every HIP translation unit built here.
"""

from __future__ import annotations

import os
import subprocess

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
SOURCES = [
    os.path.join(PKG_DIR, "csrc", "paged_decode_attention.hip"),
    os.path.join(PKG_DIR, "csrc", "rope_paged_kv.hip"),
    os.path.join(PKG_DIR, "csrc", "loom_hip_bridge.cpp"),
    os.path.join(PKG_DIR, "csrc", "loom_hip_views.cpp"),
]
LIB_PATH = os.path.join(PKG_DIR, "_build", "libloom_hip.so")
PROBE_SOURCE = os.path.join(PKG_DIR, "csrc", "hbm_probe.hip")
PROBE_LIB_PATH = os.path.join(PKG_DIR, "_build", "libloom_hip_probe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
OFFLOAD_ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{os.path.join(REPO_DIR, 'include')}",
]


def _run(cmd, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def _compile(sources, out: str, verbose: bool, incremental: bool = False) -> None:
    """Compile each source to an object under _build/obj, then link ``out``.

    With ``incremental`` an object newer than its source and every header is
    reused (a developer convenience); ``build()`` recompiles everything.
    """
    obj_dir = os.path.join(os.path.dirname(out), "obj")
    os.makedirs(obj_dir, exist_ok=True)
    headers = [os.path.join(REPO_DIR, "include", h) for h in os.listdir(os.path.join(REPO_DIR, "include"))]
    headers += [os.path.join(PKG_DIR, "csrc", h) for h in os.listdir(os.path.join(PKG_DIR, "csrc")) if h.endswith(".h")]
    newest_header = max(os.path.getmtime(h) for h in headers)
    objects = []
    for src in sources:
        obj = os.path.join(obj_dir, os.path.basename(src) + ".o")
        objects.append(obj)
        if incremental and os.path.exists(obj) and os.path.getmtime(obj) > max(os.path.getmtime(src), newest_header):
            continue
        flags = [f for f in HIPCC_FLAGS if f != "-shared"]
        _run([HIPCC, *flags, "-c", src, "-o", obj + ".tmp"], verbose)
        os.replace(obj + ".tmp", obj)
    tmp = out + ".tmp"
    _run([HIPCC, *HIPCC_FLAGS, *objects, "-o", tmp], verbose)
    os.replace(tmp, out)


ADAPTER_SOURCES = [
    os.path.join(PKG_DIR, "csrc", "torch_adapter", name)
    for name in ("torch_ops.cpp", "attention.cpp", "rope_kv.cpp")
]
ADAPTER_LIB_PATH = os.path.join(PKG_DIR, "_build", "libloom_hip_torch.so")


def _compile_adapter(verbose: bool) -> None:
    """Host-only PyTorch Stable-ABI adapter, linked against libloom_hip.so."""
    import torch.utils.cpp_extension as ext

    torch_lib = ext.library_paths()[0]
    tmp = ADAPTER_LIB_PATH + ".tmp"
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
        "-DUSE_ROCM",  # exposes the shim's aoti_torch_get_current_cuda_stream on ROCm builds
        *[f"-I{p}" for p in ext.include_paths()],
        f"-I{os.path.join(REPO_DIR, 'include')}",
        *ADAPTER_SOURCES,
        f"-L{os.path.dirname(LIB_PATH)}", "-lloom_hip",
        f"-L{torch_lib}", "-ltorch_hip", "-ltorch_cpu", "-lc10",
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}",
        "-o", tmp,
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, ADAPTER_LIB_PATH)


WAVE_TRACE_LIB_PATH = os.path.join(PKG_DIR, "_build", "libloom_hip_wave_trace.so")


def build_wave_trace(verbose: bool = False) -> str:
    """The profiling build of the library with per-wave timeline records
    (-DLOOM_HIP_WAVE_TRACE), used by ``attnarc_amd.wave_trace``; the other
    objects are the regular ones."""
    build(verbose=verbose, incremental=True)
    obj_dir = os.path.join(os.path.dirname(LIB_PATH), "obj")
    traced = os.path.join(obj_dir, "paged_decode_attention_wave_trace.o")
    flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    _run([HIPCC, *flags, "-DLOOM_HIP_WAVE_TRACE", "-c", SOURCES[0], "-o", traced], verbose)
    others = [os.path.join(obj_dir, os.path.basename(src) + ".o") for src in SOURCES[1:]]
    tmp = WAVE_TRACE_LIB_PATH + ".tmp"
    _run([HIPCC, *HIPCC_FLAGS, traced, *others, "-o", tmp], verbose)
    os.replace(tmp, WAVE_TRACE_LIB_PATH)
    return WAVE_TRACE_LIB_PATH


def build(verbose: bool = False, incremental: bool = False) -> str:
    """Compile the kernel library, the HBM probe library and the torch adapter; returns the first's path."""
    _compile(SOURCES, LIB_PATH, verbose, incremental)
    _compile([PROBE_SOURCE], PROBE_LIB_PATH, verbose, incremental)
    _compile_adapter(verbose)
    return LIB_PATH


if __name__ == "__main__":
    import sys

    if "--wave-trace" in sys.argv:
        print(build_wave_trace(verbose=True))
    else:
        print(build(verbose=True, incremental="--incremental" in sys.argv))
