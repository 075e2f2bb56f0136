"""The bench line's roofline.traffic comes from the committed rocprofv3 FETCH_SIZE /
WRITE_SIZE table of the C2 decode (profiles/decode_kernel_c2.txt); the kernel names the
bench looks up must be the ones that table lists, or the field silently becomes null."""
import importlib.util
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_c2_traffic_table_has_the_benched_kernels():
    b = _bench()
    t = b._traffic("decode_kernel_c2", ["decode_kernel<f16,128,2>", "decode_merge_kernel<4>"])
    assert t is not None
    # the C2 launch's algorithmic bytes are 2.28 GB; counter traffic sits within 10 % above them
    assert 2.2e9 <= t <= 2.6e9, t
    src = open(os.path.join(ROOT, "bench.py")).read()
    assert '"decode_merge_kernel<4>"' in src


def test_rounding_keeps_small_errors():
    b = _bench()
    r = b._rounded({"a": 3.948807e-07, "b": 5782.0412, "c": 0.0, "d": {"e": 0.00424411}})
    assert r["a"] == 3.95e-07 and r["b"] == 5782.0412 and r["c"] == 0.0 and r["d"]["e"] == 0.00424


def test_nan_max_keeps_a_nan():
    b = _bench()
    nan = float("nan")
    err = 0.0
    for e in [1e-4, nan, 3e-4, 2e-4]:  # a NaN row in the middle of the sample
        err = b._nan_max(err, e)
    assert err != err
    err = 0.0
    for e in [1e-4, 3e-4, 2e-4]:
        err = b._nan_max(err, e)
    assert err == 3e-4
    assert b._nan_max(nan, 1.0) != b._nan_max(nan, 1.0)
