"""Malformed GGUF files against both GGUF parsers (CPU only, no GPU).

The reference feeds its loader 27 adversarial byte streams
(tests/gguf_fuzz.rs) and expects an Err from each, never a panic, abort or
hang; its parser unit tests (src/model/gguf.rs:629-745) add a round trip and
three rejections.  Here every case runs through

* libvtq_runtime's parser (vtqrt_parse, the code vtqrt_load runs before it
  touches a device), and
* the oracle's independent restatement (vtqo_gguf_parse),

and the two must return the same status and text.  The status and text are
also pinned to what the reference's code path returns for that input
(src/model/gguf.rs: Cursor :483-617, parse :305-421, bytes_for_numel
:144-214), so a parser that fails in the wrong place fails the test.

ASan: the parsers are rebuilt with -fsanitize=address,undefined (and a 256 MiB
allocation cap) and run over every case plus seeded mutations of a valid
model file, so an out-of-bounds read, an arithmetic overflow or an allocation
sized by an untrusted count ends the run with a report.
"""
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

import oracle
import vtq
from vtq import runtime, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MAX = 2**64 - 1

# GGUF value-type tags (src/model/gguf.rs:60-74)
U32, I32, F32, STRING, ARRAY, U64 = 4, 5, 6, 8, 9, 10
MALFORMED, TRUNCATED, OVERFLOW, INTERNAL, NOT_IMPL = (vtq.E_MALFORMED, vtq.E_TRUNCATED, vtq.E_OVERFLOW,
                                                      vtq.E_INTERNAL, vtq.E_NOT_IMPLEMENTED)


def s(text):
    b = text.encode()
    return struct.pack("<Q", len(b)) + b


def header(version, tensors, meta):
    return b"GGUF" + struct.pack("<IQQ", version, tensors, meta)


def tensor_info(name, dims, ggml_type, offset):
    return s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) + \
        struct.pack("<IQ", ggml_type, offset)


def pad32(b):
    return b + b"\0" * (-len(b) % 32)


def kv_u32(key, v):
    return s(key) + struct.pack("<II", U32, v)


# ---- tests/gguf_fuzz.rs, case by case: (input, status, text) ----
FUZZ = {
    "empty_input": (b"", TRUNCATED, "gguf: read past end"),
    "truncated_magic_2": (b"GG", TRUNCATED, "gguf: read past end"),
    "truncated_magic_3": (b"GGU", TRUNCATED, "gguf: read past end"),
    "bad_magic": (b"XXXX" + struct.pack("<IQQ", 3, 0, 0), MALFORMED, "gguf: bad magic (not 'GGUF')"),
    "truncated_after_magic": (b"GGUF", TRUNCATED, "gguf: read past end"),
    "truncated_tensor_count": (b"GGUF" + struct.pack("<I", 3) + b"\0\0\0", TRUNCATED, "gguf: read past end"),
    "truncated_metadata_count": (b"GGUF" + struct.pack("<IQ", 3, 0) + b"\0" * 4, TRUNCATED, "gguf: read past end"),
    "tensor_count_max_does_not_allocate_or_hang": (header(3, MAX, 0), TRUNCATED, "gguf: read past end"),
    "metadata_count_max_does_not_hang": (header(3, 0, MAX), TRUNCATED, "gguf: read past end"),
    "metadata_key_truncated": (header(3, 0, 1) + struct.pack("<Q", 64), TRUNCATED, "gguf: read past end"),
    "metadata_string_over_cap": (header(3, 0, 1) + struct.pack("<Q", 2 << 20), MALFORMED,
                                 "gguf: string length > 1 MiB"),
    "unknown_metadata_value_type": (header(3, 0, 1) + s("k") + struct.pack("<I", 999), MALFORMED,
                                    "gguf: unknown value type"),
    "nested_array_rejected": (header(3, 0, 1) + s("arr") + struct.pack("<IIQ", ARRAY, ARRAY, 1), MALFORMED,
                              "gguf: nested arrays not supported"),
    "array_len_overflow_fixed_elem": (header(3, 0, 1) + s("arr") + struct.pack("<IIQ", ARRAY, U32, MAX), OVERFLOW,
                                      "gguf: array byte total overflow"),
    "array_fixed_elem_past_eof": (header(3, 0, 1) + s("arr") + struct.pack("<IIQ", ARRAY, U32, 4), TRUNCATED,
                                  "gguf: array past end of buffer"),
    "array_of_strings_len_max": (header(3, 0, 1) + s("arr") + struct.pack("<IIQ", ARRAY, STRING, MAX), TRUNCATED,
                                 "gguf: read past end"),
    "array_string_len_past_eof": (header(3, 0, 1) + s("arr") + struct.pack("<IIQQ", ARRAY, STRING, 1, 1 << 40),
                                  TRUNCATED, "gguf: array string past end"),
    "tensor_rank_too_high": (header(3, 1, 0) + s("t") + struct.pack("<I", 9), MALFORMED,
                             "gguf: tensor rank > 8 (sanity bound)"),
    "tensor_dims_product_overflows": (header(3, 1, 0) + tensor_info("t", [MAX, 2], 0, 0), OVERFLOW,
                                      "gguf: shape product overflows u64"),
    "tensor_dims_truncated": (header(3, 1, 0) + s("t") + struct.pack("<IQ", 4, 8), TRUNCATED, "gguf: read past end"),
    "tensor_numel_not_block_aligned": (pad32(header(3, 1, 0) + tensor_info("t", [33], 2, 0)) + b"\0" * 4096,
                                       MALFORMED, "gguf: Q4_0 tensor numel not a multiple of 32"),
    "tensor_unsupported_ggml_type": (pad32(header(3, 1, 0) + tensor_info("t", [32], 20, 0)) + b"\0" * 4096,
                                     MALFORMED, "gguf: byte size unknown for unsupported ggml_type"),
    "tensor_offset_past_eof": (pad32(header(3, 1, 0) + tensor_info("t", [4], 0, MAX // 2)) + b"\0" * 64, TRUNCATED,
                               "gguf: tensor extends past end of file"),
    "tensor_offset_overflow_add": (pad32(header(3, 1, 0) + tensor_info("t", [32], 0, MAX)) + b"\0" * 128, OVERFLOW,
                                   "gguf: tensor offset overflow"),
    "tensor_data_truncated": (pad32(header(3, 1, 0) + tensor_info("t", [1024], 0, 0)), TRUNCATED,
                              "gguf: tensor extends past end of file"),
    "alignment_zero_no_divide_by_zero": (header(3, 0, 1) + kv_u32("general.alignment", 0), MALFORMED,
                                         "gguf: general.alignment is zero"),
}
for _v in (0, 1, 4, 99, 2**32 - 1):  # unsupported_versions
    FUZZ[f"unsupported_version_{_v}"] = (header(_v, 0, 0), MALFORMED, "gguf: unsupported version (only v2/v3 supported)")

# ---- src/model/gguf.rs unit tests (rejections) ----
FUZZ["parser_rejects_bad_magic"] = (b"XXXXversion", MALFORMED, "gguf: bad magic (not 'GGUF')")
FUZZ["parser_rejects_unsupported_version"] = (header(99, 0, 0), MALFORMED,
                                              "gguf: unsupported version (only v2/v3 supported)")
FUZZ["parser_rejects_truncated_header"] = (b"GGUF\x03\x00\x00", TRUNCATED, "gguf: read past end")

# ---- crafted offsets, shapes and counts past the reference's own cases ----
FUZZ["tensor_end_overflow"] = (pad32(header(3, 1, 0) + tensor_info("t", [1 << 61], 0, 1 << 63)), OVERFLOW,
                               "gguf: tensor end overflow")
FUZZ["f32_byte_size_overflow"] = (pad32(header(3, 1, 0) + tensor_info("t", [1 << 31, 1 << 31], 0, 0)), OVERFLOW,
                                  "gguf: F32 byte size overflow")
# (numel / 256) * 144 and * 210 cannot exceed u64; (numel / 32) * 34 can
FUZZ["q8_0_byte_size_overflow"] = (pad32(header(3, 1, 0) + tensor_info("t", [2**64 - 32], 8, 0)), OVERFLOW,
                                   "gguf: Q8_0 byte size overflow")
FUZZ["q6_k_numel_not_multiple"] = (pad32(header(3, 1, 0) + tensor_info("t", [300], 14, 0)) + b"\0" * 1024,
                                   MALFORMED, "gguf: Q6_K tensor numel not a multiple of 256")
FUZZ["non_utf8_key"] = (header(3, 0, 1) + struct.pack("<Q", 2) + b"\xc3\x28", MALFORMED, "gguf: non-UTF8 string")
FUZZ["bad_array_elem_type"] = (header(3, 0, 1) + s("arr") + struct.pack("<IIQ", ARRAY, 13, 1), MALFORMED,
                               "gguf: bad array elem type")
FUZZ["array_of_strings_overflow_len"] = (header(3, 0, 1) + s("arr") + struct.pack("<IIQQ", ARRAY, STRING, 1, MAX),
                                         OVERFLOW, "gguf: array string overflow")
FUZZ["tensor_name_truncated"] = (header(3, 1, 0) + struct.pack("<Q", 10) + b"abc", TRUNCATED, "gguf: read past end")


def _parsers(blob, level):
    return runtime.parse(blob, level)[:2], oracle.gguf_parse(blob, level)


@pytest.mark.parametrize("name", sorted(FUZZ))
def test_reference_fuzz_case(name):
    blob, code, text = FUZZ[name]
    (rrc, rmsg), (orc, omsg) = _parsers(blob, 0)
    assert (rrc, rmsg) == (code, text), f"runtime parser on {name}"
    assert (orc, omsg) == (code, text), f"oracle parser on {name}"
    # the model level starts with the same parse
    assert _parsers(blob, 1) == ((code, text), (code, text))


def test_minimal_valid_file_still_parses():
    """gguf_fuzz.rs minimal_valid_file_still_parses: a header with no
    tensors and no metadata is a valid GGUF; as a model it has no
    general.architecture (Config::from_gguf's first error)."""
    blob = header(3, 0, 0)
    assert _parsers(blob, 0) == ((0, ""), (0, ""))
    want = (INTERNAL, "gguf: missing 'general.architecture' metadata")
    assert _parsers(blob, 1) == (want, want)


def test_parser_roundtrips_synthetic_file():
    """gguf.rs parser_roundtrips_synthetic_file: string, u32 and f32-array
    metadata, an F32 [4, 32] and a Q4_0 [32, 32] tensor."""
    buf = header(3, 2, 3) + s("general.architecture") + struct.pack("<I", STRING) + s("llama")
    buf += kv_u32("llama.embedding_length", 288)
    buf += s("tokenizer.ggml.scores") + struct.pack("<IIQff", ARRAY, F32, 2, 1.0, 2.0)
    buf += tensor_info("token_embd.weight", [4, 32], 0, 0) + tensor_info("blk.0.attn_q.weight", [32, 32], 2, 512)
    buf = pad32(buf) + np.arange(128, dtype=np.float32).tobytes() + b"\xaa" * 576
    assert _parsers(buf, 0) == ((0, ""), (0, ""))
    # one byte short: the Q4_0 tensor runs past the end
    want = (TRUNCATED, "gguf: tensor extends past end of file")
    assert _parsers(buf[:-1], 0) == (want, want)


# ---------------------------------------------------------------- models

SMALL = dict(dim=256, hidden=512, layers=2, heads=4, kv_heads=2, vocab=64, ctx=16, rope_theta=10000.0, rms_eps=1e-5)


def _model_blob(**kw):
    return synth.llama_gguf(dict(SMALL, **kw.pop("cfg", {})), 77, **kw)


def _with_meta(blob, key, vtype, payload):
    """The same model file with one more metadata pair appended to the
    metadata section (the tensor table and data shift, offsets stay valid
    relative to the aligned data base)."""
    raw = bytes(blob)
    n_t, n_kv = struct.unpack_from("<QQ", raw, 8)
    # walk the metadata to its end
    pos = 24
    for _ in range(n_kv):
        (kl,) = struct.unpack_from("<Q", raw, pos)
        pos += 8 + kl
        (vt,) = struct.unpack_from("<I", raw, pos)
        pos += 4
        if vt == STRING:
            (sl,) = struct.unpack_from("<Q", raw, pos)
            pos += 8 + sl
        else:
            pos += {U32: 4, I32: 4, F32: 4, U64: 8}[vt]
    meta_end = pos
    # the tensor table follows; its records are kept, the data re-aligned
    for _ in range(n_t):
        (nl,) = struct.unpack_from("<Q", raw, pos)
        pos += 8 + nl
        (nd,) = struct.unpack_from("<I", raw, pos)
        pos += 4 + 8 * nd + 4 + 8
    data = raw[(pos + 31) // 32 * 32:]
    head = raw[:8] + struct.pack("<QQ", n_t, n_kv + 1) + raw[24:meta_end] + s(key) + struct.pack("<I", vtype) + \
        payload + raw[meta_end:pos]
    return pad32(head) + data


def test_valid_model_parses_to_its_config():
    blob = _model_blob()
    rc, msg, dims = runtime.parse(blob, 1)
    assert (rc, msg) == (0, "")
    assert dims == (256, 512, 2, 4, 2, 64, 16)
    assert oracle.gguf_parse(blob, 1) == (0, "")


@pytest.mark.parametrize("key,payload,want", [
    # usize metadata above INT_MAX: refused before any allocation it would size
    ("llama.block_count", struct.pack("<Q", 1 << 31), (NOT_IMPL, "vtq: model dimension above INT_MAX")),
    ("llama.context_length", struct.pack("<Q", MAX), (NOT_IMPL, "vtq: model dimension above INT_MAX")),
    # INT_MAX layers: the table is walked only while the tensors exist
    ("llama.block_count", struct.pack("<Q", 2**31 - 1), (INTERNAL, "gguf: required Llama tensor not found")),
    # a zero head count (the reference divides by it while stepping)
    ("llama.attention.head_count", struct.pack("<Q", 0),
     (NOT_IMPL, "vtq: unsupported head layout (heads and kv_heads must tile dim)")),
])
def test_model_counts_are_checked(key, payload, want):
    # a repeated key keeps its last value (BTreeMap::insert), so appending overrides
    blob = _with_meta(_model_blob(), key, U64, payload)
    assert _parsers(blob, 0) == ((0, ""), (0, ""))
    assert _parsers(blob, 1) == (want, want)


def test_wrong_dtype_norm_and_bias_are_rejected():
    # general.architecture given a non-string value: Config::from_gguf's first error
    blob = _with_meta(_model_blob(), "general.architecture", U32, struct.pack("<I", 7))
    want = (INTERNAL, "gguf: missing 'general.architecture' metadata")
    assert _parsers(blob, 1) == (want, want)


def test_load_rejects_malformed_files_before_touching_a_device():
    """vtqrt_load runs the parse on the host first: every malformed case is
    refused with the reference's status and text, without a GPU (this test
    runs on the CPU image, where any device call would fail differently)."""
    for name in sorted(FUZZ):
        blob, code, text = FUZZ[name]
        with pytest.raises(vtq.VtqError) as e:
            runtime.Model(np.frombuffer(blob, dtype=np.uint8) if blob else np.zeros(0, np.uint8))
        assert (e.value.code, e.value.message) == (code, text), name


def _mutants(n=400, seed=2024):
    """Seeded mutations of a valid model file: truncations, byte flips in the
    header, and extreme values written over its u64 / u32 fields."""
    base = bytes(_model_blob(cfg=dict(layers=1, vocab=8)))
    hdr_end = 2048
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        b = bytearray(base)
        kind = i % 4
        if kind == 0:
            b = b[: int(rng.integers(0, len(base)))]
        elif kind == 1:
            for _ in range(int(rng.integers(1, 6))):
                b[int(rng.integers(0, hdr_end))] = int(rng.integers(0, 256))
        elif kind == 2:
            p = int(rng.integers(0, hdr_end - 8))
            vals = [MAX, MAX // 2, 1 << 63, 1 << 40, 2**31, 0]
            b[p:p + 8] = struct.pack("<Q", vals[int(rng.integers(0, len(vals)))])
        else:
            p = int(rng.integers(0, hdr_end - 4))
            vals = [2**32 - 1, 2**31, 9, 13, 20, 0]
            b[p:p + 4] = struct.pack("<I", vals[int(rng.integers(0, len(vals)))])
        out.append(bytes(b))
    return out


def test_mutated_models_agree_between_parsers():
    seen = set()
    for i, blob in enumerate(_mutants()):
        for level in (0, 1):
            r, o = _parsers(blob, level)
            assert r == o, f"mutant {i} level {level}: runtime {r} oracle {o}"
            seen.add(r[0])
    # the mutations reach every kind of outcome
    assert {0, MALFORMED, TRUNCATED} <= seen


def _build_asan(tmp):
    cxx, cc = shutil.which("g++"), shutil.which("gcc")
    if not cxx or not cc:
        pytest.skip("g++ / gcc not available")
    san = ["-g", "-O1", "-fno-omit-frame-pointer", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-static-libasan", "-static-libubsan"]
    objs = []
    for src in ("vtq_oracle.c", "vtq_oracle_libm.c", "vtq_oracle_blake3.c", "vtq_oracle_e2e.c"):
        obj = os.path.join(tmp, src + ".o")
        subprocess.run([cc, "-std=c11", "-ffp-contract=off", "-fno-builtin", *san, "-c",
                        os.path.join(ROOT, "oracle", src), "-o", obj], check=True)
        objs.append(obj)
    exe = os.path.join(tmp, "gguf_fuzz_driver")
    subprocess.run([cxx, "-std=c++17", *san, os.path.join(ROOT, "tests", "native", "gguf_fuzz_driver.cpp"),
                    os.path.join(ROOT, "vitni-tensor_amd", "csrc", "vtq_gguf.cpp"), *objs, "-lm", "-lpthread",
                    "-o", exe], check=True)
    return exe


def test_parsers_under_address_sanitizer(tmp_path):
    exe = _build_asan(str(tmp_path))
    cases = [FUZZ[k][0] for k in sorted(FUZZ)] + [header(3, 0, 0), bytes(_model_blob())] + _mutants(200, seed=7)
    paths = []
    for i, blob in enumerate(cases):
        p = tmp_path / f"case{i:04d}.gguf"
        p.write_bytes(blob)
        paths.append(str(p))
    # the ASan runtime is linked statically, so it needs no place in the
    # dynamic library order
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:max_allocation_size_mb=256:allocator_may_return_null=0:"
                                        "verify_asan_link_order=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe, *paths], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    lines = r.stdout.splitlines()
    assert len(lines) == 2 * len(cases)
    for ln in lines:
        rc_r, rc_o, rest = ln.split(" ", 2)
        msg_r, msg_o = rest.split(" | ", 1)
        assert (rc_r, msg_r) == (rc_o, msg_o), ln
