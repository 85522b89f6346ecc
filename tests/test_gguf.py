"""GGUF ingestion (include/m4_gguf.h), on the host.

The loader checks follow the reference's own suite (tests/test_gguf_loader.mm:
129-340: corrupt magic, header fields, metadata, tensor table, PrismML Q2_0
extraction with the reserved code 3, disk == buffer, missing tensors).  The
layout conversions into router blocks are pinned against closed forms:
GGML-standard Q4_K (the ggml block_q4_K layout, restated below from ggml's
published format: no GGML source is vendored in the reference) on a
hand-derived block and on random blocks; MLX g64 against MLX's definition
w = scale q + bias.  Every converted tensor is decoded by the oracle's pinned
router dequantizer.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest

import gguf
import synth


# --------------------------------------------------------------------------
# A GGUF writer for fixtures (test infrastructure)
# --------------------------------------------------------------------------

def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _val(t: int, v) -> bytes:
    if t == gguf.ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_val(et, i) for i in items)
    fmt = {gguf.UINT8: "<B", gguf.INT8: "<b", gguf.UINT16: "<H", gguf.INT16: "<h", gguf.UINT32: "<I",
           gguf.INT32: "<i", gguf.FLOAT32: "<f", gguf.BOOL: "<?", gguf.UINT64: "<Q", gguf.INT64: "<q",
           gguf.FLOAT64: "<d"}
    return _s(v) if t == gguf.STRING else struct.pack(fmt[t], v)


def make_gguf(kv: list, tensors: list, alignment: int = 32, version: int = 3, magic: bytes = b"GGUF") -> bytes:
    """kv: [(key, type, value)]; tensors: [(name, dims, ggml_type, data bytes)]."""
    head = magic + struct.pack("<IQQ", version, len(tensors), len(kv))
    for k, t, v in kv:
        head += _s(k) + struct.pack("<I", t) + _val(t, v)
    off, body = 0, b""
    for name, dims, t, data in tensors:
        head += _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", t, off)
        pad = (-len(data)) % alignment
        body += data + b"\0" * pad
        off += len(data) + pad
    head += b"\0" * ((-len(head)) % alignment)
    return head + body


def prism_fixture(K: int, N: int, scale: float, alignment: int = 32, magic: bytes = b"GGUF") -> bytes:
    """tests/test_gguf_loader.mm:43-127: one PrismML Q2_0 tensor whose byte i
    packs the codes (i, i+1, i+2, i+3) % 4."""
    d = np.array([scale], np.float16).tobytes()
    codes = bytes(((i % 4) | (((i + 1) % 4) << 2) | (((i + 2) % 4) << 4) | (((i + 3) % 4) << 6)) for i in range(32))
    data = (d + codes) * (K * N // 128)
    kv = [("general.architecture", gguf.STRING, "prism"), ("general.alignment", gguf.UINT32, alignment),
          ("prism.block_count", gguf.UINT32, 16)]
    return make_gguf(kv, [("model.layers.0.mlp.gate.weight", [K, N], gguf.GGML_PRISM_Q2_0, data)], alignment,
                     magic=magic)


@pytest.fixture(scope="module")
def lib(libpath):
    return gguf.library(libpath)


# --------------------------------------------------------------------------
# Loader (tests/test_gguf_loader.mm)
# --------------------------------------------------------------------------

def test_rejects_bad_magic_and_version(lib):
    ld = gguf.GGUFLoader()
    assert not ld.parse_from_buffer(prism_fixture(256, 16, 0.025, magic=b"BAD!"))
    assert not ld.is_open()
    for v in (1, 4):
        assert not ld.parse_from_buffer(make_gguf([], [], version=v))
    assert not ld.parse_from_buffer(b"GGUF")  # shorter than the header


def test_header_metadata_and_tensor_table(lib):
    K, N, align = 256, 16, 64
    ld = gguf.GGUFLoader()
    assert ld.parse_from_buffer(prism_fixture(K, N, 0.025, align))
    assert ld.is_open() and ld.version() == 3 and ld.tensor_count() == 1 and ld.metadata_count() == 3
    assert ld.alignment() == align and ld.tensor_data_offset() % align == 0
    assert ld.get_string_metadata("general.architecture") == "prism"
    assert ld.get_uint32_metadata("general.alignment") == align
    assert ld.get_uint32_metadata("prism.block_count") == 16
    assert ld.get_uint32_metadata("missing", 7) == 7 and not ld.has_metadata("missing")
    info = ld.get_tensor_info("model.layers.0.mlp.gate.weight")
    assert info.n_dims == 2 and info.dims == [K, N] and info.type == 100 and info.offset == 0
    assert ld.tensor_names() == ["model.layers.0.mlp.gate.weight"]
    assert ld.get_tensor_info("nope") is None and ld.get_tensor_raw_data("nope") is None
    assert ld.get_tensor_raw_data("model.layers.0.mlp.gate.weight") is not None


def test_every_metadata_value_type(lib):
    kv = [("u8", gguf.UINT8, 250), ("i8", gguf.INT8, -5), ("u16", gguf.UINT16, 65000), ("i16", gguf.INT16, -300),
          ("u32", gguf.UINT32, 4_000_000_000), ("i32", gguf.INT32, -70000), ("f32", gguf.FLOAT32, 1.5),
          ("b", gguf.BOOL, True), ("s", gguf.STRING, "héllo"), ("u64", gguf.UINT64, 2 ** 40 + 3),
          ("i64", gguf.INT64, -(2 ** 40)), ("f64", gguf.FLOAT64, 0.1),
          ("arr", gguf.ARRAY, (gguf.ARRAY, [(gguf.STRING, ["a", "bc"]), (gguf.STRING, [])])),
          ("general.alignment", gguf.UINT32, 16)]
    ld = gguf.GGUFLoader()
    assert ld.parse_from_buffer(make_gguf(kv, [], alignment=16))
    got = {k: ld.get_metadata(k) for k, _, _ in kv}
    assert got["u8"] == 250 and got["i8"] == -5 and got["u16"] == 65000 and got["i16"] == -300
    assert got["u32"] == 4_000_000_000 and got["i32"] == -70000 and got["f32"] == 1.5 and got["b"] is True
    assert got["s"] == "héllo" and got["u64"] == 2 ** 40 + 3 and got["i64"] == -(2 ** 40) and got["f64"] == 0.1
    assert got["arr"] == ("array", 2)
    assert ld.get_uint64_metadata("u64") == 2 ** 40 + 3 and ld.get_uint32_metadata("i32", 9) == 9
    assert ld.alignment() == 16


def test_truncated_headers_fail_cleanly(lib):
    full = prism_fixture(128, 4, 0.5)
    ld = gguf.GGUFLoader()
    hdr_end = full.index(b"\0" * 8, 60)  # somewhere inside the tensor table
    for n in list(range(0, 64)) + list(range(64, hdr_end, 7)):
        assert not ld.parse_from_buffer(full[:n]) or n >= 24
    # a header cut inside the key/value table
    assert not ld.parse_from_buffer(full[:40])


def test_extract_q2_0_known_values_and_reserved_code(lib, oracle):
    K, N, scale = 256, 16, 0.025
    ld = gguf.GGUFLoader()
    assert ld.parse_from_buffer(prism_fixture(K, N, scale))
    blocks, k, n = ld.extract_q2_0_tensor("model.layers.0.mlp.gate.weight")
    assert (k, n) == (K, N) and blocks.shape == (K * N // 128, 34)
    assert np.all(blocks[:, 0:2].copy().view(np.float16) == np.float16(scale))
    w = oracle.dequantize(7, blocks.reshape(-1), K, N).astype(np.float64).reshape(-1, 128)
    i = np.arange(32)
    codes = np.stack([(i + j) % 4 for j in range(4)], 1).reshape(-1)  # element 4 i + j
    expect = (codes - 1.0) * float(np.float16(scale))
    np.testing.assert_array_equal(w, np.broadcast_to(np.float16(expect).astype(np.float64), w.shape))
    assert np.any(codes == 3) and np.isclose(expect[codes == 3][0], 2 * float(np.float16(scale)))
    assert ld.extract_q2_0_tensor("missing") is None


def test_disk_open_matches_buffer(lib, tmp_path):
    data = prism_fixture(384, 8, 0.0625, 32)
    p = tmp_path / "prism.gguf"
    p.write_bytes(data)
    a, b = gguf.GGUFLoader(), gguf.GGUFLoader()
    assert a.open(p) and b.parse_from_buffer(data)
    assert a.file_size() == len(data)
    xa, xb = a.extract_q2_0_tensor("model.layers.0.mlp.gate.weight"), b.extract_q2_0_tensor(
        "model.layers.0.mlp.gate.weight")
    np.testing.assert_array_equal(xa[0], xb[0])
    assert xa[1:] == xb[1:] == (384, 8)
    assert not gguf.GGUFLoader().open(tmp_path / "absent.gguf")


def test_extract_rejects_bad_element_counts_and_bounds(lib):
    ld = gguf.GGUFLoader()
    assert ld.parse_from_buffer(make_gguf([], [("t", [96, 2], 100, b"\0" * 68)]))
    assert ld.extract_q2_0_tensor("t") is None  # 192 elements: not a multiple of 128
    assert ld.parse_from_buffer(make_gguf([], [("t", [128, 4], 100, b"\0" * 34)]))
    assert ld.extract_q2_0_tensor("t") is None  # 4 blocks declared, 1 present


# --------------------------------------------------------------------------
# GGML Q4_K -> router Q4_K
# --------------------------------------------------------------------------

def ggml_pack_q4_k(d, dmin, sc, mn, codes) -> np.ndarray:
    """ggml block_q4_K bytes: d, dmin (fp16), scales[12] in ggml's
    get_scale_min_k4 packing (j < 4: sc in s[j] & 63, m in s[j + 4] & 63;
    j >= 4: low 4 bits of sc / m in s[j + 4] low / high nibble, top 2 bits in
    s[j - 4] / s[j] bits 6..7), qs[128]: 32-byte chunk c holds elements
    64 c + l (low nibble) and 64 c + 32 + l (high)."""
    n = len(d)
    out = np.zeros((n, 144), np.uint8)
    out[:, 0:2] = np.asarray(d, np.float16).view(np.uint8).reshape(n, 2)
    out[:, 2:4] = np.asarray(dmin, np.float16).view(np.uint8).reshape(n, 2)
    sc, mn = np.asarray(sc, np.uint8), np.asarray(mn, np.uint8)
    s = np.zeros((n, 12), np.uint8)
    s[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    s[:, 4:8] = (mn[:, 0:4] & 63) | ((mn[:, 4:8] >> 4) << 6)
    s[:, 8:12] = (sc[:, 4:8] & 15) | ((mn[:, 4:8] & 15) << 4)
    out[:, 4:16] = s
    c = np.asarray(codes, np.uint8).reshape(n, 4, 2, 32)
    out[:, 16:] = (c[:, :, 0, :] | (c[:, :, 1, :] << 4)).reshape(n, 128)
    return out.reshape(-1)


def ggml_dequant_q4_k_exact(d, dmin, sc, mn, codes) -> np.ndarray:
    """w = d sc_j q - dmin m_j for sub-block j = element // 32 (float64, exact)."""
    d = np.asarray(d, np.float16).astype(np.float64)[:, None]
    dm = np.asarray(dmin, np.float16).astype(np.float64)[:, None]
    j = np.arange(256) // 32
    return d * np.asarray(sc, np.float64)[:, j] * np.asarray(codes, np.float64) - dm * np.asarray(mn, np.float64)[:, j]


def test_ggml_q4_k_scale_unpacking_known_block(lib, oracle):
    """Hand-derived block: d = 1, dmin = 0.5, sc_j = 60 + j % 4 (top bits set
    for every j), m_j = 33 + 3 j, code of element e = e % 16: w = sc_j q - m_j / 2."""
    sc = np.array([[60 + j % 4 for j in range(8)]])
    mn = np.array([[33 + 3 * j for j in range(8)]])
    codes = (np.arange(256) % 16)[None, :]
    g = ggml_pack_q4_k([1.0], [0.5], sc, mn, codes)
    r = gguf.repack_ggml_q4_k(g)
    w = oracle.dequantize(2, r, 256, 1).astype(np.float64)[0]
    e = np.arange(256)
    expect = (60 + (e // 32) % 4) * (e % 16) - (33 + 3 * (e // 32)) / 2
    np.testing.assert_array_equal(w, expect)


def test_ggml_q4_k_random_blocks(lib, oracle):
    rng = np.random.default_rng(5)
    n = 96
    d = (rng.random(n) * 0.01 + 1e-4).astype(np.float16)
    dmin = (rng.random(n) * 0.01).astype(np.float16)
    sc, mn = rng.integers(0, 64, (n, 8)), rng.integers(0, 64, (n, 8))
    codes = rng.integers(0, 16, (n, 256))
    r = gguf.repack_ggml_q4_k(ggml_pack_q4_k(d, dmin, sc, mn, codes))
    got = oracle.dequantize(2, r, 256, n)
    expect = ggml_dequant_q4_k_exact(d, dmin, sc, mn, codes).astype(np.float16)  # one RNE rounding
    np.testing.assert_array_equal(got.view(np.uint16), expect.view(np.uint16))
    # the router packing of the converted block is the reference generator's (bench_universal_router.mm:70-78)
    np.testing.assert_array_equal(r.reshape(n, 144)[:, 4:16], synth._pack_q4k_scales(sc, mn))


# --------------------------------------------------------------------------
# MLX g64 -> router MLX_4BIT
# --------------------------------------------------------------------------

def test_mlx_g64_repack(lib, oracle):
    N, K = 24, 512
    w = synth.gaussian_weights(N, K, 3)
    scale, bias, packed = synth.quantize_mlx_g64(w)
    r = gguf.repack_mlx_g64(packed, scale, bias)
    np.testing.assert_array_equal(r, synth.mlx_g64_to_router_blocks(scale, bias, packed))
    q = np.stack([(packed >> np.uint32(4 * j)) & 15 for j in range(8)], -1).reshape(N, K).astype(np.float64)
    g = np.arange(K) // 64
    expect = (q * scale.astype(np.float64)[:, g] + bias.astype(np.float64)[:, g]).astype(np.float16)
    np.testing.assert_array_equal(oracle.dequantize(1, r, K, N).view(np.uint16), expect.view(np.uint16))
    with pytest.raises(ValueError):
        gguf.repack_mlx_g64(packed[:, :4], scale[:, :1], bias[:, :1])  # K = 32: not whole groups


# --------------------------------------------------------------------------
# Router weights straight from a GGUF file
# --------------------------------------------------------------------------

def test_load_router_weights_per_type(lib, oracle):
    rng = np.random.default_rng(11)
    K, N = 512, 6
    q40 = synth.random_blocks(0, N, K, 1)
    q80 = synth.random_blocks(6, N, K, 2)
    pr = synth.random_blocks(7, N, K, 3)
    n4k = N * K // 256
    sc, mn = rng.integers(0, 64, (n4k, 8)), rng.integers(0, 64, (n4k, 8))
    d, dm = (rng.random(n4k) * 0.01).astype(np.float16), (rng.random(n4k) * 0.01).astype(np.float16)
    codes = rng.integers(0, 16, (n4k, 256))
    q4k = ggml_pack_q4_k(d, dm, sc, mn, codes)
    f32 = rng.standard_normal(K * N).astype(np.float32)
    data = make_gguf([], [("a", [K, N], gguf.GGML_Q4_0, q40.tobytes()), ("b", [K, N], gguf.GGML_Q8_0, q80.tobytes()),
                          ("c", [K, N], gguf.GGML_PRISM_Q2_0_ALT, pr.tobytes()),
                          ("d", [K, N], gguf.GGML_Q4_K, q4k.tobytes()), ("e", [K, N], gguf.GGML_F32, f32.tobytes()),
                          ("f", [K + 32, N], gguf.GGML_Q4_K, q4k.tobytes())])
    ld = gguf.GGUFLoader()
    assert ld.parse_from_buffer(data)
    for name, fmt, src in (("a", 0, q40), ("b", 6, q80), ("c", 7, pr)):
        W, f, k, n = ld.load_router_weights(name)
        assert (f, k, n) == (fmt, K, N)
        np.testing.assert_array_equal(W, src)
    W, f, k, n = ld.load_router_weights("d")
    assert (f, k, n) == (2, K, N)
    expect = ggml_dequant_q4_k_exact(d, dm, sc, mn, codes).reshape(N, K).astype(np.float16)
    np.testing.assert_array_equal(oracle.dequantize(2, W, K, N).view(np.uint16), expect.view(np.uint16))
    with pytest.raises(ValueError, match="status -3"):
        ld.load_router_weights("e")  # fp32 has no router format
    with pytest.raises(ValueError, match="status -4"):
        ld.load_router_weights("f")  # K = 544 is not whole Q4_K super-blocks
