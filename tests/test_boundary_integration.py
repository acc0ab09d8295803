"""The boundary as a maintainer of the reference would bind it, compiled
without a GPU.

include/aigpu_attention.h must share a translation unit with the reference's
include/ai/gpu/DeviceABI.h (both define AiGpuCounters and the AiGpuDense*
structs, DeviceABI.h:66-72, 122-143), in either include order, as C and as
C++; the C++ wrappers of include/aigpu_device.hpp must compile beside the
reference's Device.hpp and, linked against the no-device stub, answer the
way the reference's stub does (src/gpu/Stub.cpp:18-66): false, with
"no device" as the reason. The checks that need the reference's headers
skip where /root/reference is absent (the GPU box)."""
import os
import shutil
import subprocess

import pytest

import aigpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")
REF_INC = "/root/reference/include"
needs_ref = pytest.mark.skipif(not os.path.exists(os.path.join(REF_INC, "ai", "gpu", "DeviceABI.h")),
                               reason="the reference checkout is not present")


def _compile(tmp_path, name, text, lang, extra=(), link=False, libs=()):
    src = tmp_path / f"{name}.{'c' if lang == 'c' else 'cpp'}"
    src.write_text(text)
    cc = ["gcc", "-std=c11"] if lang == "c" else ["g++", "-std=c++20"]
    out = tmp_path / (name if link else f"{name}.o")
    cmd = cc + ["-Wall", "-Wextra", "-Werror", "-I", INC] + list(extra) + [str(src), "-o", str(out)] + list(libs)
    if not link:
        cmd.insert(len(cc), "-c")
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, f"{' '.join(cmd)}\n{r.stderr}"
    return out


@pytest.mark.parametrize("lang", ["c", "c++"])
def test_header_stands_alone(tmp_path, lang):
    """Without the reference on the include path the header declares the shared types itself."""
    text = ('#include "aigpu_attention.h"\n'
            "int probe(void) { AiGpuCounters c; AiGpuDenseConfig d; (void)c; (void)d;"
            " return aigpu_available(); }\n")
    _compile(tmp_path, "alone", text, lang)


@needs_ref
@pytest.mark.parametrize("lang", ["c", "c++"])
@pytest.mark.parametrize("order", ["reference_first", "backend_first"])
def test_header_shares_a_unit_with_device_abi(tmp_path, lang, order):
    a, b = '#include "ai/gpu/DeviceABI.h"\n', '#include "aigpu_attention.h"\n'
    head = a + b if order == "reference_first" else b + a
    text = head + ("int probe(void) {\n"
                   "  AiGpuCounters c; AiGpuDenseWeight w; AiGpuPrefill p; (void)w; (void)p;\n"
                   "  aigpu_counters(&c);\n"
                   "  return aigpu_available() + aigpu_dense_supported();\n}\n")
    _compile(tmp_path, f"unit_{order}", text, lang, ["-I", REF_INC])


@needs_ref
def test_header_copied_beside_device_abi(tmp_path):
    """The layout a maintainer gets by copying the header next to DeviceABI.h."""
    gpu = tmp_path / "gpu"
    gpu.mkdir()
    shutil.copy(os.path.join(REF_INC, "ai", "gpu", "DeviceABI.h"), gpu / "DeviceABI.h")
    shutil.copy(os.path.join(INC, "aigpu_attention.h"), gpu / "aigpu_attention.h")
    text = '#include "gpu/aigpu_attention.h"\n#include "gpu/DeviceABI.h"\nint probe(void) { AiGpuCounters c; (void)c; return 0; }\n'
    src = tmp_path / "beside.c"
    src.write_text(text)
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-c", "-I", str(tmp_path), str(src), "-o",
                        str(tmp_path / "beside.o")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


WRAPPER_CALLS = r"""
#include <cstdio>
#include <cstring>
#include <string>
int main() {
    float q[8] = {}, k[8] = {}, v[8] = {}, out[8] = {};
    const bool ok = ai::gpu::attention(q, k, v, out, 1, 0, 1, 1, 8, 8);
    const std::string why = ai::gpu::lastError();
    const bool dev = ai::gpu::available();
    float state[64] = {}, a[1] = {}, b[1] = {}, alog[1] = {}, dt[1] = {};
    const bool delta = ai::gpu::gatedDeltaRule(q, k, v, a, b, alog, dt, state, out, 1, 1, 1, 8, 8);
    const bool dec = ai::gpu::decodeAttention(q, k, v, out, nullptr, nullptr, nullptr, nullptr, nullptr,
                                              1e-6f, 0.f, 0, 0, 1, 1, 8, 8, 0, 1);
    std::printf("%d %d %d %d %s\n", int(ok), int(dev), int(delta), int(dec), why.c_str());
    return 0;
}
"""


@needs_ref
@pytest.mark.parametrize("order", ["reference_first", "backend_first"])
def test_wrappers_compile_beside_device_hpp_and_call_the_stub(tmp_path, order):
    a, b = '#include "ai/gpu/Device.hpp"\n', '#include "aigpu_device.hpp"\n'
    head = a + b if order == "reference_first" else b + a
    stub_dir = os.path.dirname(aigpu.STUB)
    assert os.path.exists(aigpu.STUB), "libaigpu_stub.so not built"
    # the stub is linked under its real file name, as the reference's makefile names its backend
    exe = _compile(tmp_path, f"wrappers_{order}", head + WRAPPER_CALLS, "c++",
                   ["-I", REF_INC], link=True, libs=[aigpu.STUB, f"-Wl,-rpath,{stub_dir}"])
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split(maxsplit=4)
    ok, dev, delta, dec, why = out
    assert (ok, dev, delta, dec) == ("0", "0", "0", "0")
    assert "no device" in why
