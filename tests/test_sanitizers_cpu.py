"""The host code under the sanitizers, on the CPU.

Builds instrumented copies of the step-table extension (adana_amd/csrc/
hoststep.cpp, which reads torch's TensorImpls, writes raw pointer arrays and
runs helper threads) and of the kernel library's host code
(adana_amd/csrc/adana_mta.hip: layouts, scalars, workspace sizing, argument
checks and error messages; no kernel is launched), then runs
tests/san_driver.py against each in a child process with the sanitizer
runtime preloaded:
  * the extension with AddressSanitizer + UndefinedBehaviorSanitizer (g++),
    and again with ThreadSanitizer (the helper-thread scan);
  * the library's host code with AddressSanitizer + UndefinedBehaviorSanitizer
    (hipcc's clang; -Xarch_host keeps the instrumentation off device code).
A finding ends the child with an error report; the test fails on it."""
import os
import subprocess
import sys
import sysconfig

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "adana_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"


def _torch_flags():
    import torch
    tdir = os.path.dirname(torch.__file__)
    inc = [f"-I{sysconfig.get_paths()['include']}", f"-I{tdir}/include",
           f"-I{tdir}/include/torch/csrc/api/include"]
    libs = [f"-L{tdir}/lib", f"-Wl,-rpath,{tdir}/lib", "-ltorch_python", "-ltorch_cpu", "-lc10"]
    return inc, libs, int(torch._C._GLIBCXX_USE_CXX11_ABI)


def _gcc_runtime(name):
    path = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else None


def _clang_asan_runtime():
    res = subprocess.run(["/opt/rocm/llvm/bin/clang", "-print-file-name=libclang_rt.asan-x86_64.so"],
                         capture_output=True, text=True).stdout.strip()
    if os.path.isabs(res) and os.path.exists(res):
        return res
    rt = subprocess.run(["/opt/rocm/llvm/bin/clang", "-print-runtime-dir"], capture_output=True,
                        text=True).stdout.strip()
    for cand in (os.path.join(rt, "libclang_rt.asan-x86_64.so"),
                 os.path.join(os.path.dirname(rt), "linux", "libclang_rt.asan-x86_64.so")):
        if os.path.exists(cand):
            return cand
    return None


@pytest.fixture(scope="module")
def builds(tmp_path_factory):
    """Builds the three instrumented binaries side by side (under a minute)."""
    out = tmp_path_factory.mktemp("san")
    inc, libs, abi = _torch_flags()
    ext = sysconfig.get_config_var("EXT_SUFFIX")
    jobs = {}
    common = ["g++", "-O1", "-g", "-std=c++17", "-shared", "-fPIC", f"-D_GLIBCXX_USE_CXX11_ABI={abi}", *inc]
    for kind, flags in (("asan", ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
                                  "-fno-omit-frame-pointer"]),
                        ("tsan", ["-fsanitize=thread"])):
        d = out / kind
        d.mkdir()
        cmd = [*common, *flags, "-o", str(d / f"_hoststep{ext}"), os.path.join(CSRC, "hoststep.cpp"), *libs]
        jobs[kind] = (subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True), d)
    if os.path.exists(HIPCC):
        lib = out / "libadana_mta_asan.so"
        cmd = [HIPCC, "--offload-arch=gfx950", "-O1", "-Xarch_host", "-g", "-std=c++17", "-fPIC", "-shared",
               "-ffp-contract=off", "-fno-fast-math", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
               "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer",
               f"-I{os.path.join(ROOT, 'include')}", "-o", str(lib),
               os.path.join(CSRC, "adana_mta.hip"), os.path.join(CSRC, "adana_order_stats.hip")]
        jobs["mta"] = (subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True), lib)
    built = {}
    for kind, (proc, target) in jobs.items():
        log, _ = proc.communicate(timeout=600)
        assert proc.returncode == 0, f"{kind} build failed:\n{log[-4000:]}"
        built[kind] = str(target)
    return built


def _run(mode, target, preload, extra_env):
    env = dict(os.environ)
    env["LD_PRELOAD"] = preload
    env.update(extra_env)
    res = subprocess.run([sys.executable, os.path.join(ROOT, "tests", "san_driver.py"), mode, target],
                         capture_output=True, text=True, env=env, timeout=600, cwd=ROOT)
    report = res.stdout[-3000:] + res.stderr[-6000:]
    assert res.returncode == 0, report
    for marker in ("ERROR: AddressSanitizer", "runtime error:", "WARNING: ThreadSanitizer"):
        assert marker not in res.stderr, report
    return res.stdout


def test_hoststep_address_and_undefined(builds):
    rt = _gcc_runtime("libasan.so")
    if rt is None:
        pytest.skip("gcc's libasan is not installed")
    out = _run("hoststep", builds["asan"], rt, {
        "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=0:halt_on_error=1",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"})
    assert "hoststep: ok" in out


def test_hoststep_threads(builds):
    rt = _gcc_runtime("libtsan.so")
    if rt is None:
        pytest.skip("gcc's libtsan is not installed")
    out = _run("hoststep", builds["tsan"], rt, {"TSAN_OPTIONS": "halt_on_error=1:report_signal_unsafe=0"})
    assert "hoststep: ok" in out


def test_kernel_library_host_code(builds):
    if "mta" not in builds:
        pytest.skip("hipcc is not installed")
    rt = _clang_asan_runtime()
    if rt is None:
        pytest.skip("clang's AddressSanitizer runtime is not installed")
    out = _run("mta", builds["mta"], rt, {
        "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=0:halt_on_error=1",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"})
    assert "mta host: ok" in out
