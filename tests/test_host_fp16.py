"""The public header's host fp16 helpers (include/vkllm/vkllm_common.h), which replace the reference's bit-field
conversions of src/core/vkllm_common.h:111-186: fp16 -> fp32 re-biases the exponent field, fp32 -> fp16 truncates
the mantissa and clamps the exponent field (it does not round, and it keeps the fraction bits when it clamps).

Pinned without restating the formula where the mathematics fixes the answer: every fp16 code in the normal range,
zero and infinity widens to exactly numpy's value; every in-range fp32 value narrows to the fp16 value next to it
toward zero; narrowing a widened code gives the code back. The clamped and NaN codes are the reference's bit patterns
(src/core/vkllm_common.h:133-152 and 164-183). CPU only: the helpers are header inline functions, compiled here
with gcc into a small wrapper.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

WRAPPER = r"""
#include "vkllm/vkllm_common.h"
uint32_t to32(uint16_t h) { vkllm_fp16_pack p = {h}; float f = vkllm_fp16_to_fp32(p); uint32_t u; memcpy(&u, &f, 4); return u; }
uint16_t to16(uint32_t u) { float f; memcpy(&f, &u, 4); return vkllm_fp32_to_fp16(f).bits; }
void to32_all(uint32_t *out) { for (uint32_t h = 0; h < 65536; ++h) out[h] = to32((uint16_t)h); }
void to16_many(const uint32_t *in, uint16_t *out, size_t n) { for (size_t i = 0; i < n; ++i) out[i] = to16(in[i]); }
"""


@pytest.fixture(scope="module")
def helpers(tmp_path_factory):
    d = tmp_path_factory.mktemp("fp16")
    src, so = d / "w.c", d / "w.so"
    src.write_text(WRAPPER)
    subprocess.check_call(["gcc", "-O2", "-std=c11", "-shared", "-fPIC", "-I", os.path.join(ROOT, "include"), str(src),
                           "-o", str(so)])
    L = ctypes.CDLL(str(so))
    L.to32.restype, L.to32.argtypes = ctypes.c_uint32, [ctypes.c_uint16]
    L.to16.restype, L.to16.argtypes = ctypes.c_uint16, [ctypes.c_uint32]
    L.to32_all.argtypes = [ctypes.c_void_p]
    L.to16_many.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]

    def to32_all():
        out = np.zeros(65536, np.uint32)
        L.to32_all(out.ctypes.data)
        return out

    def to16(bits32):
        bits32 = np.ascontiguousarray(bits32, np.uint32)
        out = np.zeros(bits32.size, np.uint16)
        L.to16_many(bits32.ctypes.data, out.ctypes.data, bits32.size)
        return out

    return to32_all, to16


def test_widening_all_codes(helpers):
    to32_all, _ = helpers
    got = to32_all()
    codes = np.arange(65536, dtype=np.uint32)
    exp, frac, sign = (codes >> 10) & 31, codes & 1023, codes >> 15
    exact = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32).view(np.uint32)
    normal = (exp > 0) & (exp < 31)
    zero_or_inf = ((exp == 0) | (exp == 31)) & (frac == 0)
    assert np.array_equal(got[normal], exact[normal])
    assert np.array_equal(got[zero_or_inf], exact[zero_or_inf])
    # NaN codes: fp32 NaN with the sign kept and fraction 1 (src/core/vkllm_common.h:133-141)
    nan = (exp == 31) & (frac != 0)
    assert np.array_equal(got[nan], (sign[nan] << 31) | (255 << 23) | 1)
    # subnormal codes keep exponent field 0 and shift the fraction (src/core/vkllm_common.h:145-152): not the value
    sub = (exp == 0) & (frac != 0)
    assert np.array_equal(got[sub], (sign[sub] << 31) | (frac[sub] << 13))


def test_narrowing_truncates_in_range(helpers):
    _, to16 = helpers
    rng = np.random.default_rng(3)
    mag = np.exp2(rng.uniform(-14, 15.999, 200000)).astype(np.float32)
    x = np.concatenate([mag, -mag, np.float32([1.0, 1.0 + 2 ** -11, 1.0 + 2 ** -10 - 2 ** -23, 65504.0, 65519.0,
                                               2 ** -14, 3.0 * 2 ** -15 + 2 ** -24, 0.1, 1 / 3])])
    h = to16(x.view(np.uint32)).view(np.float16).astype(np.float32)
    assert np.all(np.sign(h) == np.sign(x))
    assert np.all(np.abs(h) <= np.abs(x))
    # the fp16 number one ulp further from zero is past x: h is x's neighbour toward zero
    with np.errstate(over="ignore"):  # the neighbour of 65504 is infinity
        up = np.nextafter(np.abs(h).astype(np.float16), np.float16(np.inf)).astype(np.float32)
    assert np.all(up > np.abs(x))


def test_narrowing_round_trips_every_code(helpers):
    to32_all, to16 = helpers
    codes = np.arange(65536, dtype=np.uint32)
    exp, frac = (codes >> 10) & 31, codes & 1023
    keep = ((exp > 0) & (exp < 31)) | (frac == 0)  # normal, zero and infinite codes
    back = to16(to32_all()[keep])
    assert np.array_equal(back, codes[keep].astype(np.uint16))


def test_narrowing_clamps_and_nan(helpers):
    _, to16 = helpers

    def bits(v):
        return np.float32(v).view(np.uint32)

    # below 2^-14: exponent field 0, the top ten fraction bits kept (src/core/vkllm_common.h:174-175)
    assert to16([bits(2 ** -20 * 1.5)])[0] == (1 << 9)
    assert to16([bits(-2 ** -30)])[0] == 0x8000
    # 2^16 and above: exponent field 31 with the fraction bits, so 2^16 is infinity and 1.5 * 2^16 a NaN code
    # (src/core/vkllm_common.h:176-177)
    assert to16([bits(2.0 ** 16)])[0] == 0x7C00
    assert to16([bits(-1.5 * 2 ** 16)])[0] == 0xFC00 | (1 << 9)
    assert to16([bits(np.inf)])[0] == 0x7C00
    # NaN: exponent 31, fraction 1, sign kept (src/core/vkllm_common.h:164-171)
    assert to16([0x7FC00000])[0] == 0x7C01
    assert to16([0xFFC00001])[0] == 0xFC01
