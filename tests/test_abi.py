"""C-ABI checks that need no GPU: the library loads, exports every entry point the public
headers declare, and rejects bad arguments without touching a device."""
import ctypes
import os
import re

import pytest

import edge_maskgit_amd as ema

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mgh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ema.lib()
    declared = _declared("mgh.h")
    assert declared, "no declarations parsed"
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    assert sorted(ema.MGH_SYMBOLS) == declared


def test_version():
    assert ema.lib().mgh_version() == 1


def test_null_context_errors_without_device():
    L = ema.lib()
    assert L.mgh_last_error(None) == b"null context"
    assert L.mgh_gemm_q(None, 8, None, 1, 64, None, None, None, 1, None, 0, None, None) == -1
    assert L.mgh_quantize_act_q8(None, None, 1, 32, None, None, None) == -1
    assert L.mgh_sync(None) == -1
    L.mgh_destroy(None)      # no-op


def test_package_has_no_cpu_fallback():
    # The shipped package must not import the oracle or any CPU compute path.
    src_dir = os.path.join(ROOT, "edge_maskgit_amd")
    for dirpath, _, files in os.walk(src_dir):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h", ".hpp")):
                txt = open(os.path.join(dirpath, f)).read()
                assert "import oracle" not in txt and "from oracle" not in txt, f
                assert "mg_oracle" not in txt, f


def _declared_mgr():
    text = open(os.path.join(ROOT, "include", "mgr.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mgr_[a-z0-9_]+)\s*\(", text)))


def test_runtime_library_exports_every_declared_symbol():
    from edge_maskgit_amd import runtime
    lib = runtime.lib()
    declared = _declared_mgr()
    assert declared
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    assert sorted(runtime.MGR_SYMBOLS) == declared


def test_runtime_errors_without_device(tmp_path):
    from edge_maskgit_amd import runtime
    with pytest.raises(ema.MghError):
        runtime.gguf_info(str(tmp_path / "missing.gguf"))
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"NOTAGGUF" * 8)
    with pytest.raises(ema.MghError):
        runtime.gguf_info(str(bad))


def test_every_mfma_kernel_builds_with_vgpr_results():
    """Every kernel source that issues MFMAs is compiled with -amdgpu-mfma-vgpr-form (results in
    VGPRs; without it the unrolled loops rotate their accumulators through the AGPRs), and the
    packed-fp32 feature is off for all of them."""
    import glob
    from edge_maskgit_amd import build
    srcs = sorted(glob.glob(os.path.join(build.CSRC, "*.hip")))
    mfma = [os.path.basename(s) for s in srcs if "__builtin_amdgcn_mfma" in open(s).read()]
    assert mfma
    for name in mfma:
        assert name in build.KERNEL_SOURCES, name
        assert "-amdgpu-mfma-vgpr-form" in build.EXTRA_FLAGS.get(name, []), name
    flags = " ".join(build.HIP_FLAGS)
    assert "-target-feature -Xclang -packed-fp32-ops" in flags
