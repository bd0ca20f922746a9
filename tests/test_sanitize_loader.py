"""The GGUF loader and the upload staging under the address, undefined-behaviour and thread
sanitizers, on the CPU (tests/sanitize: host/fllm_host.cpp's open_gguf / fllmh_load_gguf and
csrc/staging.hpp over a stand-in device whose copies run on a thread of their own).

GgufReader / GgufModelLoader.LoadAsync (GgufReader.cs:37-167, GgufModelLoader.cs:336-372): a GGUF
file written by the package's writer is loaded cold (page cache dropped), warm, and by two threads
at once on one context; every tensor's "device" bytes equal the file's, the slack after each is
cleared; files cut in the header or in the tensor data, a bad magic and a missing path fail with
FLLM_E_MODEL_LOAD. The default file is the Qwen2 vocabulary on one narrow layer (190 MB, a
155 MB embedding through five staging chunks); FLLM_SANITIZE_GGUF_CONFIG names another config
(qwen2-7b-q5k: the 7.1 GB file of the Qwen2-7B bench, about 4 minutes under ASan).
"""
import os
import shutil
import subprocess

import pytest

from dotnetfoundryllm_amd.configs import CONFIGS
from dotnetfoundryllm_amd.gguf import write_synthetic_gguf

HERE = os.path.dirname(os.path.abspath(__file__))
SAN = os.path.join(HERE, "sanitize")


@pytest.fixture(scope="module")
def binaries(tmp_path_factory):
    if shutil.which("g++") is None or shutil.which("make") is None:
        pytest.skip("g++ / make not found")
    out = str(tmp_path_factory.mktemp("sanitize_build"))
    r = subprocess.run(["make", "-C", SAN, f"OUT={out}"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    return os.path.join(out, "load_check_asan"), os.path.join(out, "load_check_tsan")


@pytest.fixture(scope="module")
def gguf_file(tmp_path_factory):
    name = os.environ.get("FLLM_SANITIZE_GGUF_CONFIG", "test-qwen2-v152k")
    d = tmp_path_factory.mktemp("sanitize_gguf")
    path = str(d / f"{name}.gguf")
    write_synthetic_gguf(path, CONFIGS[name])
    return path, str(d)


def run(binary, path, scratch, env_extra):
    env = dict(os.environ, **env_extra)
    r = subprocess.run([binary, path, scratch], capture_output=True, text=True, timeout=3000, env=env)
    text = r.stdout + r.stderr
    return r.returncode, text


def test_loader_under_address_and_ub_sanitizers(binaries, gguf_file):
    rc, text = run(binaries[0], *gguf_file, {"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0",
                                             "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1"})
    print(text)
    assert rc == 0 and "load check ok" in text, text
    assert "AddressSanitizer" not in text and "runtime error" not in text and "LeakSanitizer" not in text


def test_loader_under_thread_sanitizer(binaries, gguf_file):
    rc, text = run(binaries[1], *gguf_file, {"FLLM_STUB_DMA_DELAY_US": "50", "TSAN_OPTIONS": "halt_on_error=1"})
    print(text)
    assert rc == 0 and "load check ok" in text, text
    assert "ThreadSanitizer" not in text
