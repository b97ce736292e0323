"""Build the gfx950 libraries in-tree with hipcc (no JIT, no site-packages install).

  libmgh.so      HIP kernels + the C ABI of include/mgh.h
  libmg_hip.so   C++ host side: the mg tensor/graph API, GGUF loader, transformer graph
                 builder and HipRuntime (include/mg-tensor.hpp, include/mg-hip.hpp)

Objects go to edge_maskgit_amd/_build/, libraries to edge_maskgit_amd/lib/.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(PKG, "host")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "lib")

ARCH = "gfx950"
# Packed fp32 VALU ops (v_pk_*_f32) are disabled for all device code: forms of them have given
# silently wrong results on this hardware, and the compiler would otherwise emit them from plain
# fp32 code.
HIP_FLAGS = ["--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wno-unused-command-line-argument"]

KERNEL_SOURCES = ["k_quant_act.hip", "k_gemm_i8.hip",
                  "k_pack_w.hip", "k_gemm_qp.hip", "k_layernorm.hip", "k_flash_attn.hip",
                  "k_gemm_f32.hip", "k_glue.hip", "k_ops.hip", "k_vqgan.hip", "k_conv_i8.hip", "noalloc.hip", "k_decode.hip", "k_gemm_fc.hip", "mgh_api.cpp"]
# Per-source extra flags. Every MFMA kernel keeps its MFMA results in VGPRs: the int8 GEMMs'
# per-block scale arithmetic then reads them without v_accvgpr_read copies, and in the
# unrolled K loops of the FC GEMM and the attention's tile loops the accumulators no longer
# rotate through the AGPRs at each loop back edge (4-28 v_accvgpr moves per iteration in the
# FC kernels with 64-row weight tiles, up to ~200 per attention kernel), with the same
# occupancy and fewer registers.
_VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
EXTRA_FLAGS = {src: _VGPR_FORM for src in ("k_gemm_i8.hip", "k_gemm_qp.hip", "k_conv_i8.hip", "k_gemm_fc.hip",
                                           "k_flash_attn.hip", "k_gemm_f32.hip", "k_vqgan.hip")}
# C++ host runtime (graph API mirror, GGUF loader, transformer builder, HipRuntime, mgr C ABI):
# plain host code over the libmgh C ABI, compiled with g++ into lib/libmg_hip.so.
HOST_SOURCES = ["mg-tensor.cpp", "mg-model.cpp", "mg-transformer.cpp", "mg-vqgan.cpp", "mg-hip.cpp", "mgr_api.cpp"]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-parameter"]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found (ROCm install expected at /opt/rocm)")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")
    if out.strip() and verbose:
        print(out)


def _stale(target, deps):
    if not os.path.exists(target):
        return True
    t = os.path.getmtime(target)
    return any(os.path.getmtime(d) > t for d in deps)


def _headers():
    hs = []
    for d in (CSRC, HOST, os.path.join(ROOT, "include")):
        if os.path.isdir(d):
            hs += [os.path.join(d, f) for f in os.listdir(d) if f.endswith((".h", ".hpp"))]
    return hs


def build(verbose: bool = False, force: bool = True) -> None:
    """Compile every source (force=True rebuilds everything, as __graft_entry__.build()
    requires); force=False only rebuilds stale objects."""
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIB, exist_ok=True)
    cc = hipcc()
    hdrs = _headers()
    inc = ["-I" + os.path.join(ROOT, "include"), "-I" + CSRC, "-I" + HOST]
    jobs = []
    objs = []
    for src in KERNEL_SOURCES:
        s = os.path.join(CSRC, src)
        o = os.path.join(OBJ, src + ".o")
        if force or _stale(o, [s] + hdrs):
            jobs.append([cc, *HIP_FLAGS, *EXTRA_FLAGS.get(src, []), *inc, "-c", s, "-o", o])
        objs.append(o)
    hobjs = []
    for src in HOST_SOURCES:
        s = os.path.join(HOST, src)
        o = os.path.join(OBJ, src + ".o")
        if force or _stale(o, [s] + hdrs):
            jobs.append([shutil.which("g++") or "g++", *HOST_FLAGS, *inc, "-c", s, "-o", o])
        hobjs.append(o)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        for f in [ex.submit(_run, j, verbose) for j in jobs]:
            f.result()
    libmgh = os.path.join(LIB, "libmgh.so")
    tmp = libmgh + ".tmp"
    _run([cc, *HIP_FLAGS, "-shared", "-o", tmp, *objs], verbose)
    os.replace(tmp, libmgh)
    if HOST_SOURCES:
        libmg = os.path.join(LIB, "libmg_hip.so")
        tmp = libmg + ".tmp"
        _run([shutil.which("g++") or "g++", "-shared", "-o", tmp, *hobjs, "-L" + LIB, "-lmgh",
              "-Wl,-rpath,$ORIGIN"], verbose)
        os.replace(tmp, libmg)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv, force="--force" in sys.argv or "-f" in sys.argv)
