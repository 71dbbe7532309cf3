"""The ONNX decoder built for the host alone under AddressSanitizer and UndefinedBehaviorSanitizer
(tests/native/onnx_loader_fuzz.cpp) and run over seeded mutations of mnist-8.onnx and of a BERT
encoder layer: every damaged model loads or is refused with the decoder's own status, with no read
outside the model buffer, no leak and no undefined arithmetic. CPU only; skipped where g++ lacks
the sanitizer runtimes."""
import os
import shutil
import subprocess

import pytest

from bert_layer import bert_layer

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


@pytest.fixture(scope="module")
def fuzzer(tmp_path_factory):
    if not shutil.which("g++"):
        pytest.skip("g++ not found")
    d = tmp_path_factory.mktemp("asan")
    exe = str(d / "onnx_loader_fuzz")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
           "-fno-omit-frame-pointer", "-I/opt/rocm/include", "-D__HIP_PLATFORM_AMD__",
           os.path.join(ROOT, "onnx_amd", "csrc", "lx_onnx.cpp"), os.path.join(HERE, "native", "onnx_loader_fuzz.cpp"),
           "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    if r.returncode and "asan" in r.stderr.lower() and "cannot find" in r.stderr.lower():
        pytest.skip("sanitizer runtimes missing: " + r.stderr[-300:])
    assert r.returncode == 0, r.stderr[-3000:]
    bert = d / "bert_layer.onnx"
    bert.write_bytes(bert_layer(1, 8, 3)[0])
    return exe, [os.path.join(HERE, "golden", "mnist-8.onnx"), str(bert)]


@pytest.mark.parametrize("seed", [7])
def test_decoder_under_sanitizers(fuzzer, seed):
    exe, models = fuzzer
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe, str(seed), "400", *models], capture_output=True, text=True, timeout=900, env=env)
    assert r.returncode == 0, r.stderr[-4000:]
    loaded, refused = (int(v) for v in r.stdout.split()[1::2])
    assert loaded > 0 and refused > 0 and loaded + refused == 400
