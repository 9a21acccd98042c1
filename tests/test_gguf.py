"""GGUF reading and RWKV-7 ingestion (CPU).

The reference reads GGUF through the third-party ``gguf`` package, absent
here, and holds no GGUF file, so nothing of the reference reads these files;
the checks pin the container to the published GGUF v3 layout instead:

* a file assembled byte by byte in this test (struct.pack, not the module's
  writer) is parsed as the layout says: metadata of every type, tensor shapes
  (ne reversed), the aligned data section, every readable tensor type;
* the block formats decode to their published closed forms, computed here
  element by element (Q4_0: d ((q & 15) - 8) for the low nibbles then the high
  nibbles; Q4_1: d q + m; Q8_0: d q; BF16: the upper 16 bits of an fp32);
* writer -> reader round trips (custom alignment, string arrays);
* RWKV-7: GGUF (llama.cpp names, every matrix logical (out, in)) -> v3 blob
  equals the blob written directly from the same weights, fp32 and INT4, with
  a tied head and with per-layer ranks; a BF16 file equals the blob of the
  weights rounded to bfloat16 by torch; the reference's own C runtime loads
  the converted blob and its step matches the oracle bit for bit.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

import oracle
from sunnynet_amd.gguf import GGMLType, GGUFFile, gguf_to_rwkv7_blob, rwkv7_to_gguf_tensors, write_gguf
from sunnynet_amd.rwkv7 import RWKV_TINY, init_rwkv7, pack_rwkv7_blob


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _f16(x) -> bytes:
    return np.float16(x).tobytes()


def test_hand_assembled_file_parses_per_spec(tmp_path):
    rng = np.random.default_rng(0)
    kv = [
        (_s("a.u8") + struct.pack("<IB", 0, 200), 200),
        (_s("a.i8") + struct.pack("<Ib", 1, -5), -5),
        (_s("a.u16") + struct.pack("<IH", 2, 60000), 60000),
        (_s("a.i16") + struct.pack("<Ih", 3, -30000), -30000),
        (_s("a.u32") + struct.pack("<II", 4, 4000000000), 4000000000),
        (_s("a.i32") + struct.pack("<Ii", 5, -2000000000), -2000000000),
        (_s("a.f32") + struct.pack("<If", 6, 0.25), 0.25),
        (_s("a.bool") + struct.pack("<I?", 7, True), True),
        (_s("a.str") + struct.pack("<I", 8) + _s("hello"), "hello"),
        (_s("a.arr") + struct.pack("<IIQ", 9, 5, 3) + struct.pack("<3i", 1, -2, 3), [1, -2, 3]),
        (_s("a.sarr") + struct.pack("<IIQ", 9, 8, 2) + _s("x") + _s("yz"), ["x", "yz"]),
        (_s("a.u64") + struct.pack("<IQ", 10, 2**40), 2**40),
        (_s("a.i64") + struct.pack("<Iq", 11, -2**40), -2**40),
        (_s("a.f64") + struct.pack("<Id", 12, 1.5), 1.5),
    ]
    # Tensors: F32 (3,5), F16 (4,), BF16 (2,2), Q8_0 (32,), Q4_0 (2,32), Q4_1 (32,).
    f32 = rng.standard_normal((3, 5)).astype(np.float32)
    f16 = rng.standard_normal(4).astype(np.float16)
    bf_bits = rng.integers(0, 2**16, 4).astype(np.uint16)
    bf_bits[(bf_bits & 0x7F80) == 0x7F80] &= 0x3FFF          # finite values only
    q8_d, q8_q = np.float16(0.03), rng.integers(-128, 128, 32).astype(np.int8)
    q4_d = [np.float16(0.5), np.float16(-0.125)]
    q4_qs = [rng.integers(0, 256, 16).astype(np.uint8) for _ in range(2)]
    q41_d, q41_m, q41_qs = np.float16(0.2), np.float16(-1.0), rng.integers(0, 256, 16).astype(np.uint8)
    datas = [
        ("t.f32", (5, 3), 0, f32.tobytes()),
        ("t.f16", (4,), 1, f16.tobytes()),
        ("t.bf16", (2, 2), 30, bf_bits.tobytes()),
        ("t.q8", (32,), 8, _f16(q8_d) + q8_q.tobytes()),
        ("t.q4", (32, 2), 2, b"".join(_f16(d) + q.tobytes() for d, q in zip(q4_d, q4_qs))),
        ("t.q41", (32,), 3, _f16(q41_d) + _f16(q41_m) + q41_qs.tobytes()),
    ]
    align = 32
    infos, data, off = b"", b"", 0
    for name, ne, t, raw in datas:
        infos += _s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        infos += struct.pack("<IQ", t, off)
        pad = (-len(raw)) % align
        data += raw + b"\0" * pad
        off += len(raw) + pad
    head = b"GGUF" + struct.pack("<IQQ", 3, len(datas), len(kv)) + b"".join(k for k, _ in kv) + infos
    head += b"\0" * ((-len(head)) % align)
    path = tmp_path / "hand.gguf"
    path.write_bytes(head + data)

    g = GGUFFile(path)
    assert g.version == 3
    for (raw, want), key in zip(kv, [k for k in g.meta]):
        assert g.meta[key] == want, key
    assert g.tensors["t.f32"].shape == (3, 5)
    assert np.array_equal(g.tensor("t.f32"), f32)
    assert np.array_equal(g.tensor("t.f16"), f16.astype(np.float32))
    bf_want = np.array([struct.unpack("<f", struct.pack("<I", int(b) << 16))[0] for b in bf_bits],
                       np.float32).reshape(2, 2)
    assert np.array_equal(g.tensor("t.bf16"), bf_want)
    assert np.array_equal(g.tensor("t.q8"), np.float32(q8_d) * q8_q.astype(np.float32))
    want = np.empty((2, 32), np.float32)
    for r in range(2):
        for j in range(16):
            want[r, j] = np.float32(q4_d[r]) * ((int(q4_qs[r][j]) & 15) - 8)
            want[r, j + 16] = np.float32(q4_d[r]) * ((int(q4_qs[r][j]) >> 4) - 8)
    assert np.array_equal(g.tensor("t.q4"), want)
    want41 = np.array([np.float32(q41_d) * (int(q41_qs[j % 16]) & 15 if j < 16 else int(q41_qs[j % 16]) >> 4)
                       + np.float32(q41_m) for j in range(32)], np.float32)
    assert np.allclose(g.tensor("t.q41"), want41, rtol=0, atol=1e-6)


def test_writer_roundtrip_alignment_and_strings(tmp_path):
    rng = np.random.default_rng(1)
    a = rng.standard_normal((7, 3)).astype(np.float32)
    b = rng.standard_normal((4, 8)).astype(np.float32)
    toks = ["<s>", "\\x00", "héllo", "\\xe4\\xb8\\xad", "中"]
    path = tmp_path / "w.gguf"
    write_gguf(path, {"general.architecture": "test", "n": 7, "x": 0.5, "tokenizer.ggml.tokens": toks},
               {"a": a, "b.weight": (GGMLType.F16, (8, 4), b.astype(np.float16).tobytes())}, alignment=64)
    g = GGUFFile(path)
    assert g.alignment == 64 and all(t.offset % 64 == 0 for t in g.tensors.values())
    assert g.meta["general.architecture"] == "test" and g.meta["n"] == 7 and g.meta["x"] == 0.5
    assert np.array_equal(g.tensor("a"), a)
    assert np.array_equal(g.tensor("b"), b.astype(np.float16).astype(np.float32))
    # The reference's rule (runtime/gguf.py:90-103): latin-1 bytes with \xNN
    # escapes undone; text outside latin-1 falls back to UTF-8.
    assert g.tokens() == [b"<s>", b"\x00", b"h\xe9llo", "中".encode("utf-8"), "中".encode("utf-8")]


def _rwkv_gguf(tmp_path, w, name, ggml_type=GGMLType.F32, tied=False):
    cfg = w.cfg
    meta = {"general.architecture": "rwkv7", "rwkv7.block_count": cfg.layers,
            "rwkv7.embedding_length": cfg.dim, "rwkv7.wkv.head_size": cfg.head_size,
            "rwkv7.feed_forward_length": cfg.ff, "rwkv7.attention.layer_norm_epsilon": cfg.eps,
            "tokenizer.ggml.tokens": [f"t{i}" for i in range(cfg.vocab)]}
    path = tmp_path / name
    write_gguf(path, meta, rwkv7_to_gguf_tensors(w, ggml_type, tied=tied))
    return path


@pytest.mark.parametrize("int4", [False, True])
@pytest.mark.parametrize("tied", [False, True])
def test_rwkv7_gguf_to_blob_equals_direct_blob(tmp_path, int4, tied):
    w = init_rwkv7(RWKV_TINY, 4)
    if tied:
        w.head = w.embed.copy()
    path = _rwkv_gguf(tmp_path, w, "m.gguf", tied=tied)
    assert gguf_to_rwkv7_blob(path, int4=int4) == pack_rwkv7_blob(w, int4=int4)


def test_rwkv7_bf16_gguf_is_the_bf16_rounded_model(tmp_path):
    w = init_rwkv7(RWKV_TINY, 5)
    path = _rwkv_gguf(tmp_path, w, "bf.gguf", GGMLType.BF16)

    def bf(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).float().numpy()

    w.layers = [{k: bf(v) for k, v in L.items()} for L in w.layers]
    for k in ("en_w", "en_b", "on_w", "on_b", "embed", "head"):
        setattr(w, k, bf(getattr(w, k)))
    assert gguf_to_rwkv7_blob(path, int4=False) == pack_rwkv7_blob(w)


def test_rwkv7_ragged_ranks_run_on_the_reference_runtime(tmp_path):
    """Layer 1 with other LoRA ranks: the rank table comes from the file's
    shapes, and the reference's C runtime steps the converted blob exactly as
    the oracle does."""
    if not oracle.ref_available():
        pytest.skip("reference C build (oracle/_ref) not present")
    w = init_rwkv7(RWKV_TINY, 6)
    rng = np.random.default_rng(7)
    D = w.cfg.dim
    for k, r in (("w", 32), ("g", 16)):
        w.layers[1][k + "1"] = (rng.standard_normal((r, D)) / np.sqrt(D)).astype(np.float32)
        w.layers[1][k + "2"] = (rng.standard_normal((D, r)) * 0.5 / np.sqrt(r)).astype(np.float32)
    path = _rwkv_gguf(tmp_path, w, "rag.gguf")
    blob = gguf_to_rwkv7_blob(path, int4=False)
    hdr = struct.unpack_from("<10i", blob)
    ranks = [struct.unpack_from("<4i", blob, 44 + 16 * i) for i in range(w.cfg.layers)]
    assert hdr[7] == max(r[3] for r in ranks) and ranks[1] == (32, 64, 32, 16) and ranks[0] == w.cfg.ranks
    bp = tmp_path / "rag.bin"
    bp.write_bytes(blob)
    ref = oracle.RefRk(bp, w.cfg.vocab)
    orc = oracle.RkOracle(blob)
    for t in (3, 77, 400, 9):
        assert np.array_equal(ref.step(t), orc.step([t])[0])


def test_reader_rejects_malformed_files(tmp_path):
    """Wrong magic, an unsupported version, a misaligned tensor offset and
    tensor data past the end of the file are refused, not read."""
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + struct.pack("<IQQ", 3, 0, 0))
    with pytest.raises(ValueError, match="not a GGUF"):
        GGUFFile(bad)
    bad.write_bytes(b"GGUF" + struct.pack("<IQQ", 9, 0, 0))
    with pytest.raises(ValueError, match="version"):
        GGUFFile(bad)
    head = b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + _s("t") + struct.pack("<IQIQ", 1, 8, 0, 4)
    bad.write_bytes(head + b"\0" * ((-len(head)) % 32) + b"\0" * 64)
    with pytest.raises(ValueError, match="not aligned"):
        GGUFFile(bad)
    head = b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + _s("t") + struct.pack("<IQIQ", 1, 1000, 0, 0)
    bad.write_bytes(head + b"\0" * ((-len(head)) % 32) + b"\0" * 64)
    with pytest.raises(ValueError, match="past the end"):
        GGUFFile(bad)


def test_converter_cli_writes_the_blob(tmp_path):
    from sunnynet_amd.gguf import main
    w = init_rwkv7(RWKV_TINY, 8)
    src = _rwkv_gguf(tmp_path, w, "cli.gguf")
    dst = tmp_path / "cli.bin"
    assert main([str(src), str(dst), "--f32"]) == 0
    assert dst.read_bytes() == pack_rwkv7_blob(w)
    assert main([str(src), str(dst)]) == 0
    assert dst.read_bytes() == pack_rwkv7_blob(w, int4=True)


@pytest.mark.gpu
def test_rwkv7_gguf_ragged_ranks_on_the_gpu_handle(gpu, tmp_path):
    """A GGUF file converted with ragged per-layer LoRA ranks, loaded by the
    HIP handle (snhip_rk_load): every step's logits equal the oracle's (B=2
    runs the exact one-launch kernel on two grid slices, which follows the
    reference's rounding order)."""
    import torch

    from sunnynet_amd.runtime.rwkv7 import HipRwkv7
    w = init_rwkv7(RWKV_TINY, 6)
    rng = np.random.default_rng(7)
    D = w.cfg.dim
    for k, r in (("w", 32), ("g", 16)):
        w.layers[1][k + "1"] = (rng.standard_normal((r, D)) / np.sqrt(D)).astype(np.float32)
        w.layers[1][k + "2"] = (rng.standard_normal((D, r)) * 0.5 / np.sqrt(r)).astype(np.float32)
    path = _rwkv_gguf(tmp_path, w, "rag.gguf")
    for int4 in (False, True):
        blob = gguf_to_rwkv7_blob(path, int4=int4)
        bp = tmp_path / f"rag{int(int4)}.bin"
        bp.write_bytes(blob)
        hm = HipRwkv7(bp, max_batch=2)
        orc = oracle.RkOracle(blob, batch=2)
        for t in ((3, 77), (400, 9), (12, 500)):
            tt = np.array(t, np.int32)
            a = hm.step_batch(torch.from_numpy(tt).to(gpu)).cpu().numpy()
            assert np.array_equal(a, orc.step(tt)), (int4, t)
        hm.close()
