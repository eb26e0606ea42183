"""bench.py's contract on the host: one GPU only, and every native timing loop it binds exists."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_bench_library_exports():
    sys.path.insert(0, ROOT)
    import bench
    L = bench.bench_lib()   # binds argtypes: a missing export raises AttributeError here
    for name in ("bn_moe_decode", "bn_moe_ffn", "bn_moe_ffn_tokens", "bn_gemv", "bn_gemm", "bn_moe_grouped",
                 "bn_copy", "bn_read", "bn_set_ramp_ms"):
        assert getattr(L, name) is not None
    L.bn_set_ramp_ms(100.0)   # host-only setter
