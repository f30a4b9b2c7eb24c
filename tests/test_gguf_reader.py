"""The library's GGUF reader (vkllm.c_amd/csrc/gguf.cpp) on crafted files, on the CPU, built with AddressSanitizer and
UndefinedBehaviorSanitizer (tests/gguf_probe.cpp drives it). The reference opens models through gguf-tools'
gguf_open and returns VKLLM_ERR_ARGS when that fails (src/models/vkllm_models_llama2.c:265-270); this reader must
reject every malformed file the same way, with no read outside the mapping, and parse well-formed ones exactly.
"""
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

import gguf_util as G

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "vkllm.c_amd", "csrc")


@pytest.fixture(scope="module")
def probe(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is not installed")
    exe = str(tmp_path_factory.mktemp("gguf_probe") / "gguf_probe")
    subprocess.run([gxx, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
                    "-fno-sanitize-recover=all", "-I", CSRC, os.path.join(ROOT, "tests", "gguf_probe.cpp"),
                    os.path.join(CSRC, "gguf.cpp"), "-o", exe], check=True)

    def run(*paths):
        # the environment is passed on as it is (any preloaded library included); AddressSanitizer is told not to
        # insist on coming first in the library order
        env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=23:verify_asan_link_order=0",
                   UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1:exitcode=24")
        r = subprocess.run([exe, *map(str, paths)], capture_output=True, text=True, env=env, timeout=60)
        assert r.returncode == 0, f"sanitizer report or crash (exit {r.returncode}):\n{r.stderr[-3000:]}"
        return r.stdout.splitlines()

    return run


def _s(b):
    b = b.encode() if isinstance(b, str) else b
    return struct.pack("<Q", len(b)) + b


def _kv_u32(key, v):
    return _s(key) + struct.pack("<II", G.U32, v)


def _tinfo(name, ne, ty, offset):
    return _s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne) + \
        struct.pack("<IQ", ty, offset)


def raw_file(path, kvs=(), infos=(), n_tensors=None, n_kv=None, data=b"", align=32, version=3, magic=b"GGUF"):
    """A GGUF file from raw key/value and tensor-info records, its data section padded to `align`."""
    head = magic + struct.pack("<IQQ", version, len(infos) if n_tensors is None else n_tensors,
                               len(kvs) if n_kv is None else n_kv)
    body = head + b"".join(kvs) + b"".join(infos)
    body += b"\0" * ((-len(body)) % align)
    with open(path, "wb") as f:
        f.write(body + data)
    return path


def test_well_formed_file_parses_exactly(probe, tmp_path):
    rng = np.random.default_rng(0)
    a = rng.standard_normal((3, 5)).astype(np.float16)
    b = rng.standard_normal(7).astype(np.float32)
    path = tmp_path / "ok.gguf"
    G.write(str(path), [("tokenizer.ggml.tokens", (G.ARRAY, G.STRING), ["<unk>", "a", "▁b"]),
                        ("llama.block_count", G.U32, 1)],
            [("a", [5, 3], G.GGML_F16, a), ("b", [7], G.GGML_F32, b)])
    out = probe(path)
    assert out[0] == "OK 3 2"  # general.alignment + the two keys
    ta = out[1].split()
    tb = out[2].split()
    assert ta[:9] == ["T", "a", "5", "3", "1", "1", "1", "0", str(a.nbytes)]
    assert int(ta[9]) == int(np.frombuffer(a.tobytes(), np.uint8).sum())
    assert tb[:9] == ["T", "b", "7", "1", "1", "1", "0", "32", str(b.nbytes)]
    assert int(tb[9]) == int(np.frombuffer(b.tobytes(), np.uint8).sum())
    assert out[3] == f"S tokenizer.ggml.tokens 3 {len('<unk>') + len('a') + len('▁b'.encode())}"


@pytest.mark.parametrize("what", ["missing", "empty", "short", "magic", "version"])
def test_rejects_unreadable_headers(probe, tmp_path, what):
    path = tmp_path / f"{what}.gguf"
    if what == "empty":
        path.write_bytes(b"")
    elif what == "short":
        path.write_bytes(b"GGUF" + b"\3\0\0\0" + b"\0" * 8)
    elif what == "magic":
        raw_file(path, magic=b"GGML")
    elif what == "version":
        raw_file(path, version=1)
    want = {"missing": "ERR cannot open file", "empty": "ERR file too small", "short": "ERR file too small",
            "magic": "ERR bad magic", "version": "ERR unsupported GGUF version"}[what]
    assert probe(path) == [want]


def test_every_truncation_of_a_model_file_is_rejected(probe, tmp_path):
    """A complete small model file cut at every length inside its header, and at points inside its data section."""
    full = tmp_path / "model.gguf"
    G.llama_model(str(full), ["<unk>", "<s>", "</s>", "a", "b"], [0, 0, 0, -1, -2], dim=32, n_head=2, ffn=64)
    blob = full.read_bytes()
    assert probe(full)[0].startswith("OK ")
    cuts = list(range(24, 1200, 7)) + [len(blob) - 1, len(blob) - 33, len(blob) // 2]
    paths = []
    for n in cuts:
        p = tmp_path / f"cut{n}.gguf"
        p.write_bytes(blob[:n])
        paths.append(p)
    out = probe(*paths)
    assert len(out) == len(cuts)
    for n, line in zip(cuts, out):
        assert line.startswith("ERR "), f"cut at {n} bytes of {len(blob)}: {line}"


@pytest.mark.parametrize("case", ["offset_past_eof", "offset_wraps", "count_overflow", "data_past_eof", "dims",
                                  "alignment", "string_length", "array_length", "kv_count", "tensor_count"])
def test_rejects_malformed_records(probe, tmp_path, case):
    path = tmp_path / f"{case}.gguf"
    data = b"\1" * 64
    t_ok = _tinfo("w", [4, 4], G.GGML_F16, 0)
    if case == "offset_past_eof":
        raw_file(path, infos=[_tinfo("w", [4], G.GGML_F16, 4096)], data=data)
        want = "ERR tensor offset past end of file: w"
    elif case == "offset_wraps":
        # offset + size wraps past 2^64 back into the file
        raw_file(path, infos=[t_ok, _tinfo("x", [16], G.GGML_F16, 2 ** 64 - 16)], data=data)
        want = "ERR tensor offset past end of file: x"
    elif case == "count_overflow":
        raw_file(path, infos=[_tinfo("w", [2 ** 32, 2 ** 32, 2], G.GGML_F16, 0)], data=data)
        want = "ERR tensor element count overflows: w"
    elif case == "data_past_eof":
        raw_file(path, infos=[_tinfo("w", [64], G.GGML_F16, 0)], data=data)  # 128 bytes, 64 present
        want = "ERR tensor data past end of file: w"
    elif case == "dims":
        raw_file(path, infos=[_tinfo("w", [1, 1, 1, 1, 1], G.GGML_F16, 0)], data=data)
        want = "ERR truncated or malformed header"
    elif case == "alignment":
        raw_file(path, kvs=[_kv_u32("general.alignment", 1 << 30)], infos=[t_ok], data=data)
        want = "ERR alignment larger than the file"
    elif case == "string_length":
        raw_file(path, kvs=[struct.pack("<Q", 2 ** 63) + b"key"], data=data)
        want = "ERR truncated or malformed header"
    elif case == "array_length":
        raw_file(path, kvs=[_s("tokenizer.ggml.tokens") + struct.pack("<IIQ", G.ARRAY, G.STRING, 2 ** 60) + _s("a")],
                 data=data)
        want = "ERR truncated or malformed header"
    elif case == "kv_count":
        raw_file(path, kvs=[_kv_u32("a", 1)], n_kv=2 ** 63, data=data)
        want = "ERR truncated or malformed header"
    else:
        raw_file(path, infos=[t_ok], n_tensors=2 ** 62, data=data)
        want = "ERR truncated or malformed header"
    assert probe(path) == [want]


def test_non_float_tensors_span_to_the_next_tensor(probe, tmp_path):
    """Encodings other than F32/F16 (which the reference reads as fp16 bytes) get the bytes up to the next tensor's
    offset, or to the end of the file, never past it."""
    path = tmp_path / "q.gguf"
    raw_file(path, infos=[_tinfo("q", [32], 8, 0), _tinfo("r", [32], 8, 64)], data=bytes(range(96)))
    out = probe(path)
    assert out[0] == "OK 0 2"
    assert out[1].split()[7:9] == ["0", "64"]
    assert out[2].split()[7:9] == ["64", "32"]
