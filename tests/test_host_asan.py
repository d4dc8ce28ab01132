"""The host layer under AddressSanitizer + UBSan, built from the product's own host sources
with gcc and run for a few seeds; any sanitizer report fails the test:
  tests/asan/qload_fuzz.c    random safetensors header mutations through sgl_qst_open /
                             get_raw / sgl_qlinear_probe
  tests/asan/qweight_fuzz.c  random (small, huge, negative) shapes through every
                             sgl_qlinear_create* / dequant validation, and sgl_qcfg_from_json"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


HOST = os.path.join(ROOT, "sglang.c_amd", "host")
HARNESSES = {
    "qload_fuzz.c": ["qload.c", "qjson.c"],
    "qweight_fuzz.c": ["qweight.c", "qjson.c", "qlog.c", "quant.c"],
}


@pytest.mark.parametrize("harness", sorted(HARNESSES))
def test_host_layer_clean_under_asan(tmp_path, harness):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    exe = tmp_path / "fuzz"
    src = [os.path.join(ROOT, "tests", "asan", harness)] + \
        [os.path.join(HOST, f) for f in HARNESSES[harness]]
    cmd = ["gcc", "-std=c11", "-g", "-O1", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer",
           "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(ROOT, "sglang.c_amd", "csrc"),
           "-I" + os.path.join(ROOT, "sglang.c_amd", "host"),
           '-DASAN_FUZZ_PATH="%s"' % (tmp_path / "f.st"), *src, "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0 and "sanitize" in r.stderr:
        pytest.skip("sanitizer runtime not available: " + r.stderr[-200:])
    assert r.returncode == 0, r.stderr[-2000:]
    for seed in ("1", "7"):
        run = subprocess.run([str(exe), seed], capture_output=True, text=True, timeout=300,
                             env=dict(os.environ, ASAN_OPTIONS="detect_leaks=1"))
        assert run.returncode == 0 and "runtime error" not in run.stderr, run.stderr[-3000:]
        assert "asan fuzz done" in run.stdout
