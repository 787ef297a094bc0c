"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer (CPU only; SURVEY's auxiliary
plan): the C oracle's own test file against a sanitizer build of oracle/ssm_oracle.c, the
library's checkpoint parser (ssmjs_amd/csrc/ssmw.cpp, the host code behind
ssm_model_load_weights' CHECKPOINT_INVALID contract) driven with valid, truncated, oversized,
corrupted and randomly mutated images, and the Node-API addon (ssmjs_amd/napi/ssm_napi.cc,
built here with g++ and the sanitizers) driven through its argument parsing and error paths
under Node. The HIP kernels are not built with sanitizers (GPU code); any report makes the run
fail (halt_on_error)."""
import json
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _asan_runtime():
    gcc = shutil.which("gcc")
    if gcc is None:
        return None
    p = subprocess.run([gcc, "-print-file-name=libasan.so"], capture_output=True,
                       text=True).stdout.strip()
    return p if os.path.isabs(p) and os.path.exists(p) else None


ASAN = _asan_runtime()
needs_asan = pytest.mark.skipif(ASAN is None, reason="gcc's ASan runtime is absent")


def _san_env(**extra):
    env = dict(os.environ, LD_PRELOAD=ASAN,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    env.update(extra)
    return env


@needs_asan
def test_oracle_tests_under_asan_ubsan():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "asan"], check=True)
    lib = os.path.join(ROOT, "oracle", "libssm_oracle_asan.so")
    env = _san_env(SSM_ORACLE_LIB=lib)
    which = subprocess.run([sys.executable, "-c",
                            "from oracle import oracle as O; O.lib(); print(O._LIB_PATH)"],
                           capture_output=True, text=True, cwd=ROOT, env=env, timeout=120)
    assert which.returncode == 0, which.stderr[-2000:]
    assert which.stdout.strip() == lib
    r = subprocess.run([sys.executable, "-m", "pytest", "tests/test_oracle.py", "-q",
                        "-p", "no:cacheprovider"],
                       capture_output=True, text=True, cwd=ROOT, env=env, timeout=600)
    assert r.returncode == 0, (r.stdout[-3000:], r.stderr[-3000:])
    assert "passed" in r.stdout and "failed" not in r.stdout


@needs_asan
def test_checkpoint_parser_under_asan_ubsan(tmp_path):
    """The SSMW validator and f16 codec of ssm_model_load_weights (session.ts:393-401: a bad
    checkpoint must surface as CHECKPOINT_INVALID) over every truncation, one-byte header
    corruptions, wrapping payload sizes and 40000 random mutations (tests/ssmw_check.cpp)."""
    exe = tmp_path / "ssmw_check"
    csrc = os.path.join(ROOT, "ssmjs_amd", "csrc")
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
                    "-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-I", csrc,
                    os.path.join(ROOT, "tests", "ssmw_check.cpp"), os.path.join(csrc, "ssmw.cpp"),
                    "-o", str(exe)], check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, (r.stdout[-3000:], r.stderr[-3000:])
    assert r.stdout.startswith("ok "), r.stdout


NODE = shutil.which("node")
NODE_INC = os.environ.get("NODE_INCLUDE", "/usr/include/node")
LIB = os.path.join(ROOT, "ssmjs_amd", "libssm_hip.so")


@needs_asan
@pytest.mark.skipif(NODE is None or not os.path.exists(os.path.join(NODE_INC, "node_api.h"))
                    or not os.path.exists(LIB), reason="node, node_api.h or the library absent")
def test_addon_under_asan_ubsan(tmp_path):
    addon = tmp_path / "ssm_napi_asan.node"
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-shared", "-fPIC",
                    "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
                    "-fno-sanitize-recover=undefined", "-DNODE_GYP_MODULE_NAME=ssm_napi",
                    "-I", NODE_INC, os.path.join(ROOT, "ssmjs_amd", "napi", "ssm_napi.cc"),
                    "-o", str(addon), "-L" + os.path.dirname(LIB), "-lssm_hip",
                    "-Wl,-rpath," + os.path.dirname(LIB)], check=True)
    script = tmp_path / "drive.js"
    script.write_text("""
const a = require(process.argv[2]);
const out = {};
(async () => {
  out.version = a.version();
  try { await a.ctxCreate(0); out.ctx = 'created'; } catch (e) { out.ctx = e.code; }
  try { a.forward(); } catch (e) { out.noargs = e.code; }
  try { a.ctxInfo({}); } catch (e) { out.badhandle = e.code; }
  try { a.modelCreate(null, {}, 0); } catch (e) { out.badcfg = e.code; }
  try { a.forward({}, new Uint32Array(4), 1, 4); } catch (e) { out.badmodel = e.code; }
  try { a.forward({}, 'not an array', 1, 4); } catch (e) { out.badids = e.code; }
  console.log(JSON.stringify(out));
})();
""")
    # no device: every GPU call ends at GPU_UNAVAILABLE, the argument checks run before it
    r = subprocess.run([NODE, str(script), str(addon)], capture_output=True, text=True,
                       cwd=ROOT, env=_san_env(SSM_HIP_FAULT="nodevice"), timeout=120)
    assert r.returncode == 0, r.stderr[-3000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["version"] >= 1
    assert out["ctx"] == "GPU_UNAVAILABLE"
    for k in ("noargs", "badhandle", "badcfg", "badmodel", "badids"):
        assert out[k] == "UNKNOWN", (k, out)
