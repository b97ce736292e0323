"""bench.py's command-line contract on the CPU: more than one GPU is refused with a message
(this build measures one GPU; the check runs before any device call)."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


def _bench():
    sys.path.insert(0, ROOT)
    import bench
    return bench


def test_traffic_file_is_used_only_on_the_sources_it_was_measured_on(tmp_path):
    """roofline.traffic comes from a committed rocprofv3 summary only when that summary names the
    digest of the kernel sources the bench runs; another digest gives null and the reason."""
    import json
    bench = _bench()
    d = bench.csrc_digest()
    assert len(d) == 16 and int(d, 16) >= 0
    assert bench.csrc_digest() == d                                   # deterministic
    f = tmp_path / "traffic.json"
    f.write_text(json.dumps({"traffic_bytes_per_step": 123, "csrc_sha256_16": d, "git_head": "abc",
                             "command": ["rocprofv3 ..."]}))
    t, src = bench.measured_traffic(str(f), d)
    assert t == 123 and src["git_head"] == "abc" and "stale" not in src
    t, src = bench.measured_traffic(str(f), "0" * 16)
    assert t is None and "not used" in src["stale"]
    assert bench.measured_traffic(str(tmp_path / "absent.json"), d) == (None, None)


def test_committed_traffic_files_carry_their_provenance():
    """every profiles/traffic_*.json names the git head, the kernel-source digest and the exact
    rocprofv3 commands it was measured with"""
    import glob
    import json
    files = glob.glob(os.path.join(ROOT, "profiles", "traffic_*.json"))
    assert files
    for fn in files:
        tj = json.load(open(fn))
        assert tj["git_head"] and len(tj["csrc_sha256_16"]) == 16
        assert any(c.startswith("rocprofv3 ") and "bench.py" in c for c in tj["command"])
        assert tj["traffic_bytes_per_step"] > 0
