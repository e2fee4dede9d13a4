"""GGUF reader (include/swamp_gguf.h) against an independent writer: header,
metadata conversions, tensor infos, zero-copy raw bytes and every error the
reference's GgufFile::parse returns (swamp-gguf/src/mmap.rs:34-94,
metadata.rs:117-243, tensor_info.rs:19-37).  CPU only: nothing here touches
a device."""
import math
import os

import numpy as np
import pytest

from gguf_writer import (ARRAY, BOOL, F32, F64, I8, I16, I32, I64, STRING, U8, U16, U32, U64,
                         write_gguf)

Q4_0, Q8_0, Q4_K, T_F32, T_F16, Q6_K, BF16 = 2, 8, 12, 0, 1, 14, 30


def rnd(n, seed):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8).tobytes()


def sample_tensors(pkg):
    out = []
    for i, (name, dt, shape) in enumerate([
            ("blk.0.attn_q.weight", Q4_0, [4096, 32]),
            ("blk.0.ffn_down.weight", Q8_0, [128, 3]),
            ("output.weight", Q4_K, [512, 2]),
            ("token_embd.norm", T_F32, [77]),
            ("rope.freqs", T_F16, [3, 5, 7]),
            ("blk.0.ffn_up.weight", Q6_K, [256, 4]),
            ("empty", BF16, [0, 16])]):
        n = math.prod(shape)
        out.append((name, shape, dt, rnd(pkg.gpu_lib().swamp_nbytes_for(dt, n), i)))
    return out


KV = [("general.architecture", STRING, "llama"),
      ("a.u8", U8, 200), ("a.i8", I8, -5), ("a.u16", U16, 65000), ("a.i16", I16, -300),
      ("a.u32", U32, 4000000000), ("a.i32", I32, -7), ("a.f32", F32, 1.5), ("a.bool", BOOL, True),
      ("a.u64", U64, 2 ** 40 + 3), ("a.i64", I64, -2 ** 40), ("a.f64", F64, 0.1),
      ("tok.tokens", ARRAY, (STRING, ["<s>", "</s>", "héllo"])),
      ("tok.scores", ARRAY, (F32, [0.5, -1.0])),
      ("a.dup", U32, 1), ("a.dup", U32, 2),
      ("general.alignment", U32, 64)]


@pytest.mark.parametrize("version", [1, 2, 3])
def test_round_trip(pkg, tmp_path, version):
    tensors = sample_tensors(pkg)
    path = str(tmp_path / f"v{version}.gguf")
    data_offset, offs = write_gguf(path, tensors, KV, version=version)
    with pkg.GgufFile(path) as g:
        assert g.version == version
        assert g.n_tensors() == len(tensors) and g.n_kv == len(KV)
        assert g.data_offset == data_offset and g.data_offset % 32 == 0
        assert g.file_size == os.path.getsize(path)
        for (name, shape, dt, data), off, info in zip(tensors, offs, g.tensors):
            assert (info.name, info.shape, info.dtype, info.offset) == (name, shape, dt, off)
            assert info.nbytes == len(data)
            assert g.tensor_raw_bytes(info).tobytes() == data
        assert g.tensor("output.weight").dtype == Q4_K
        assert g.tensor("missing") is None
        with pytest.raises(pkg.GpuError) as e:
            g.tensor_or_err("missing")
        assert e.value.code == pkg.ENOTFOUND
        assert g.architecture() == "llama"


def test_metadata_conversions(pkg, tmp_path):
    path = str(tmp_path / "kv.gguf")
    write_gguf(path, [], KV)
    with pkg.GgufFile(path) as g:
        assert g.meta_type("a.f64") == F64 and g.meta_type("tok.tokens") == ARRAY
        assert g.meta_type("nope") is None
        # as_u32 (metadata.rs:60-68): U8, U16, U32, I32 bit-cast
        assert g.get_u32("a.u8") == 200 and g.get_u32("a.u16") == 65000
        assert g.get_u32("a.u32") == 4000000000 and g.get_u32("a.i32") == 2 ** 32 - 7
        for key in ("a.u64", "a.i8", "a.i16", "a.f32", "a.bool", "general.architecture"):
            with pytest.raises(pkg.GpuError) as e:
                g.get_u32(key)
            assert e.value.code == pkg.ENOTFOUND, key
        # as_u64 (:70-80): also U64, I64; signed values sign-extend
        assert g.get_u64("a.u64") == 2 ** 40 + 3
        assert g.get_u64("a.i32") == 2 ** 64 - 7 and g.get_u64("a.i64") == 2 ** 64 - 2 ** 40
        # as_f32 (:82-90): F32, F64 (rounded to f32), U32, I32
        assert g.get_f32("a.f32") == 1.5
        assert g.get_f32("a.f64") == float(np.float32(0.1))
        assert g.get_f32("a.i32") == -7.0 and g.get_f32("a.u32") == float(np.float32(4e9))
        with pytest.raises(pkg.GpuError):
            g.get_f32("a.u8")
        assert g.get_str("general.architecture") == "llama"
        # a duplicate key keeps the last value (HashMap insert, mmap.rs:52-57)
        assert g.get_u32("a.dup") == 2
        # general.alignment is read as metadata but does not move the data
        # section (GGUF_ALIGNMENT = 32, mmap.rs:13, 76-79)
        assert g.get_u32("general.alignment") == 64


def test_alignment_is_32_regardless_of_key(pkg, tmp_path):
    """general.alignment is not consulted: the data section starts at the
    header end rounded up to 32 (mmap.rs:13, 76-79).  The same header
    written with 64-byte padding is read at the 32-byte position."""
    t = [("w", [32], Q8_0, rnd(34, 9))]
    for pad in range(64):  # a header whose end is 32- but not 64-aligned
        kv = [("general.alignment", U32, 64), ("pad", STRING, "x" * pad)]
        d32, _ = write_gguf(str(tmp_path / "a32.gguf"), t, kv, align=32)
        d64, _ = write_gguf(str(tmp_path / "a64.gguf"), t, kv, align=64)
        if d32 != d64:
            break
    assert d32 != d64
    with pkg.GgufFile(str(tmp_path / "a64.gguf")) as g:
        assert g.data_offset == d32 and g.tensors[0].offset == d32


def test_duplicate_tensor_names_find_first(pkg, tmp_path):
    path = str(tmp_path / "dup.gguf")
    t = [("w", [32], Q8_0, rnd(34, 1)), ("w", [64], Q8_0, rnd(68, 2))]
    write_gguf(path, t)
    with pkg.GgufFile(path) as g:
        assert g.tensor("w").index == 0 and g.tensor("w").shape == [32]


def test_zero_dims_and_empty(pkg, tmp_path):
    path = str(tmp_path / "z.gguf")
    t = [("scalar", [], T_F32, rnd(4, 3)), ("e", [0], Q4_0, b"")]
    write_gguf(path, t)
    with pkg.GgufFile(path) as g:
        assert g.tensors[0].shape == [] and g.tensors[0].nbytes == 4  # product of [] = 1
        assert g.tensors[1].nbytes == 0 and len(g.tensor_raw_bytes(g.tensors[1])) == 0


def err(pkg, path):
    with pytest.raises(pkg.GpuError) as e:
        pkg.GgufFile(path)
    return e.value.code


def test_errors(pkg, tmp_path):
    p = lambda n: str(tmp_path / n)
    assert err(pkg, p("does-not-exist.gguf")) == pkg.EIO
    open(p("empty.gguf"), "wb").close()
    assert err(pkg, p("empty.gguf")) == pkg.EIO
    write_gguf(p("magic.gguf"), [], magic=b"GGUG")
    assert err(pkg, p("magic.gguf")) == pkg.EMAGIC
    for v in (0, 4):
        write_gguf(p(f"ver{v}.gguf"), [], version=v)
        assert err(pkg, p(f"ver{v}.gguf")) == pkg.EVERSION
    t = sample_tensors(pkg)
    full, _ = write_gguf(p("full.gguf"), t, KV)
    # the file ends inside the header: UnexpectedEof -> Io
    for cut in (6, 20, 60, full - 40):
        write_gguf(p(f"cut{cut}.gguf"), t, KV, truncate=cut)
        assert err(pkg, p(f"cut{cut}.gguf")) == pkg.EIO, cut
    # unknown metadata value type and array element type: UnknownDType
    import struct
    bad_kv = struct.pack("<Q", 3) + b"bad" + struct.pack("<I", 13)
    write_gguf(p("kvtype.gguf"), [], raw_kv=bad_kv)
    assert err(pkg, p("kvtype.gguf")) == pkg.EDTYPE
    bad_arr = struct.pack("<Q", 3) + b"arr" + struct.pack("<IIQ", ARRAY, 13, 1)
    write_gguf(p("arrtype.gguf"), [], raw_kv=bad_arr)
    assert err(pkg, p("arrtype.gguf")) == pkg.EDTYPE
    nested = struct.pack("<Q", 3) + b"arr" + struct.pack("<IIQ", ARRAY, ARRAY, 0)
    write_gguf(p("nested.gguf"), [], raw_kv=nested)
    assert err(pkg, p("nested.gguf")) == pkg.EDTYPE
    # tensor dtype outside GgmlDType::from_u32 (dtype.rs:43-75)
    for code in (4, 5, 31, 1000):
        write_gguf(p(f"dt{code}.gguf"), [("w", [32], code, b"")])
        assert err(pkg, p(f"dt{code}.gguf")) == pkg.EDTYPE, code


def test_tensor_past_end_is_invalid_tensor(pkg, tmp_path):
    path = str(tmp_path / "short.gguf")
    data_offset, _ = write_gguf(path, [("w", [4096], Q4_0, rnd(2304, 5))], truncate=None)
    size = os.path.getsize(path)
    with open(path, "r+b") as f:
        f.truncate(size - 100)
    with pkg.GgufFile(path) as g:  # parse succeeds; the byte range is checked on access
        with pytest.raises(pkg.GpuError) as e:
            g.tensor_raw_bytes(g.tensors[0])
        assert e.value.code == pkg.ETENSOR


def test_raw_bytes_dequantize_like_the_oracle(pkg, orc, tmp_path):
    """The bytes handed out are the tensor's blocks: the oracle dequantizes
    them exactly as the bytes that were written."""
    path = str(tmp_path / "q.gguf")
    raws = [pkg.synth_quantized(dt, 40 + i, 0.02, 8, 512) for i, dt in enumerate((Q4_0, Q8_0, Q4_K))]
    t = [(f"m{i}", [512, 8], dt, r.tobytes()) for i, (dt, r) in enumerate(zip((Q4_0, Q8_0, Q4_K), raws))]
    write_gguf(path, t)
    with pkg.GgufFile(path) as g:
        for (name, shape, dt, data), info in zip(t, g.tensors):
            got = orc.dequantize(dt, g.tensor_raw_bytes(info), 8 * 512)
            ref = orc.dequantize(dt, np.frombuffer(data, np.uint8), 8 * 512)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
