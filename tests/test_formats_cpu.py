"""On-disk formats through the C ABI (host only, no GPU): UTH1 / UTH2
expert-blob headers against the reference's own known answers
(tensor_header.rs:567-800, expert_cache.rs:1374-1400) and the GGUF MoE
reader against synthetic files whose expert bytes the test keeps
(the reference's extraction tests, gguf_loader.rs:4104-4170,
:4382-4450, :4960-5000, do the same in memory)."""
from __future__ import annotations

import struct

import numpy as np
import pytest

import gguf_synth as gs


def uth2_bytes(d_model, d_ff, ranges, version=2, flags=1):
    """A MixedExpertHeader as to_bytes lays it out (tensor_header.rs:250-270):
    magic, u16 version, u16 count 3, u32 d_model, u32 d_ff, u32 flags, then
    24-byte records at 24 + 24 i: u8 dtype, u8 role, u64 offset @4, u64
    len @12, u32 weights @20; 128 bytes in all."""
    b = bytearray(128)
    b[0:4] = b"UTH2"
    struct.pack_into("<HHIII", b, 4, version, 3, d_model, d_ff, flags)
    for i, (dt, off, ln, w) in enumerate(ranges):
        o = 24 + 24 * i
        b[o], b[o + 1] = dt, i
        struct.pack_into("<QQI", b, o + 4, off, ln, w)
    return bytes(b)


# MixedExpertHeader::new(64, 128, Q4_0 0+18 (32 w), Q4K 18+144 (256), Q5K 162+176 (256)) of the reference tests
MIXED = [(4, 0, 18, 32), (3, 18, 144, 256), (8, 162, 176, 256)]


# -- UTH1 -------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [0, 1, 2, 3, 4, 5, 8, 9, 10])
def test_swiglu_header_roundtrip(mer, dtype):
    """roundtrip_swiglu_header + swiglu_header_quant_scale_metadata_per_dtype:
    [d_ff, d_model, 3] rank 3; Int8 advertises three scales at offset 0."""
    raw = mer.swiglu_expert_header(dtype, 512, 2048, block_align=0)
    assert len(raw) == 64 and raw[:4] == b"UTH1"
    h = mer.probe_uth(raw, 0)
    assert h.kind == 1 and h.version == 1 and h.dtype == dtype
    assert h.shape == (2048, 512, 3)
    assert (h.d_model, h.d_ff) == (512, 2048)
    assert (h.quant_scale_offset, h.quant_scale_count) == ((0, 3) if dtype == 2 else (0, 0))
    assert h.flags & 1
    # field positions, independently of the probe
    assert struct.unpack_from("<HBB4I", raw, 4) == (1, dtype, 3, 2048, 512, 3, 0)
    assert struct.unpack_from("<6I", raw, 24) == (0, 3 if dtype == 2 else 0, 16, 16, 64, 1)


def test_write_padded_aligns_payload(mer):
    raw = mer.swiglu_expert_header(mer.UthDtype.F32, 8, 16, block_align=4096)
    assert len(raw) == 4096
    assert not any(raw[64:])
    assert mer.probe_uth(raw, 4096).shape == (16, 8, 3)


def test_strip_skips_padded_prefix(mer):
    buf = mer.swiglu_expert_header(mer.UthDtype.F32, 8, 16, 4096) + b"\xab" * 64
    h, payload = mer.strip_uth(buf, 4096)
    assert h is not None and h.payload_offset == 4096
    assert len(payload) == 64 and bytes(payload) == b"\xab" * 64


def test_strip_returns_legacy_blob_unchanged(mer):
    buf = np.full(128, 0xCD, np.uint8)
    h, payload = mer.strip_uth(buf, 4096)
    assert h is None
    assert len(payload) == 128 and payload.ctypes.data == buf.ctypes.data


def test_resident_uses_configured_block_align(mer):
    """resident_uses_configured_block_align_for_uth_payload: an 8192-aligned
    header strips at 8192, not at the default 4096."""
    buf = bytearray(mer.swiglu_expert_header(mer.UthDtype.Q4_0, 32, 32, 8192))
    buf[8192:8200] = b"\x11" * 8
    buf += b"\0" * (16384 - len(buf))
    h, payload = mer.strip_uth(bytes(buf), 8192)
    assert h.payload_offset == 8192 and len(payload) == 8192 and bytes(payload[:8]) == b"\x11" * 8


@pytest.mark.parametrize("case", ["short", "version0", "version2", "rank0", "rank5", "dtype11", "prefix_past_end"])
def test_uth1_malformed_headers_read_as_legacy(mer, case):
    raw = bytearray(mer.swiglu_expert_header(mer.UthDtype.Q4_0, 32, 64, 0))
    if case == "short":
        raw = raw[:63]
    elif case == "version0":
        struct.pack_into("<H", raw, 4, 0)
    elif case == "version2":
        struct.pack_into("<H", raw, 4, 2)
    elif case == "rank0":
        raw[7] = 0
    elif case == "rank5":
        raw[7] = 5
    elif case == "dtype11":
        raw[6] = 11
    elif case == "prefix_past_end":
        raw += b"\0" * 100  # 164 bytes, but the page-aligned prefix is 4096
        assert mer.probe_uth(bytes(raw), 0) is not None
        assert mer.probe_uth(bytes(raw), 4096) is None
        return
    assert mer.probe_uth(bytes(raw), 0) is None


def test_uth1_without_page_flag_ignores_alignment(mer):
    raw = bytearray(mer.swiglu_expert_header(mer.UthDtype.Q8_0, 32, 64, 0))
    struct.pack_into("<I", raw, 44, 0)
    h = mer.probe_uth(bytes(raw) + b"\x01" * 10, 4096)
    assert h.payload_offset == 64 and h.payload_len == 10


# -- UTH2 -------------------------------------------------------------------

def test_mixed_uth2_roundtrip_and_strip(mer):
    """mixed_uth2_roundtrip_and_strip: 4096-aligned prefix, payload[0] = 0xA5,
    projection ranges as written (payload extent 338)."""
    head = uth2_bytes(64, 128, MIXED)
    file = head + b"\0" * (4096 - 128) + b"\xa5" * 338 + b"\0" * (4096 - 338)
    h, payload = mer.strip_uth(file, 4096)
    assert h.kind == 2 and h.version == 2 and h.dtype == mer.UthDtype.MIXED
    assert (h.d_model, h.d_ff) == (64, 128)
    assert h.payload_offset == 4096 and len(payload) == 4096 and payload[0] == 0xA5
    assert [(p.dtype, p.offset, p.len, p.weights) for p in h.projections] == MIXED
    assert max(p.offset + p.len for p in h.projections) == 338
    # block_align 0: no padding, payload right after the 128 bytes; the
    # header alone has no room for its ranges and is not stripped
    assert mer.probe_uth(head + b"\0" * 338, 0).payload_offset == 128
    assert mer.probe_uth(head + b"\0" * 337, 0) is None


@pytest.mark.parametrize("case", ["future_version", "count2", "overlap", "past_end", "zero_len", "mixed_dtype",
                                  "zero_d_model", "wrong_role", "dtype11", "overflow"])
def test_mixed_uth2_rejects_malformed(mer, case):
    ranges, kw = [list(r) for r in MIXED], {}
    d_model = 64
    if case == "overlap":
        ranges[1][1] = 8
    elif case == "past_end":
        ranges[2][2] = 4096 - 162 + 1
    elif case == "zero_len":
        ranges[0][2] = 0
    elif case == "mixed_dtype":
        ranges[1][0] = 10
    elif case == "dtype11":
        ranges[1][0] = 11
    elif case == "zero_d_model":
        d_model = 0
    elif case == "future_version":
        kw["version"] = 3
    elif case == "overflow":
        ranges[2][1] = 2 ** 64 - 8
    head = bytearray(uth2_bytes(d_model, 128, [tuple(r) for r in ranges], **kw))
    if case == "count2":
        struct.pack_into("<H", head, 6, 2)
    elif case == "wrong_role":
        head[24 + 24 + 1] = 2
    file = bytes(head) + b"\0" * (8192 - 128)
    # a rejected UTH2 header falls through to UTH1 ("UTH2" is not "UTH1"): legacy
    assert mer.probe_uth(file, 4096) is None
    if case == "past_end":  # one byte more payload and it fits
        assert mer.probe_uth(file + b"\0", 4096).kind == 2


def test_uth2_adjacent_ranges_are_not_overlap(mer):
    file = uth2_bytes(64, 128, [(4, 0, 10, 1), (4, 10, 10, 1), (4, 20, 10, 1)]) + b"\0" * 30
    assert mer.probe_uth(file, 0).kind == 2
    assert mer.probe_uth(file, 4096) is None  # the page-aligned prefix lies past the end


def test_probe_accepts_empty_and_tensor_buffers(mer):
    import torch

    assert mer.probe_uth(b"", 4096) is None
    t = torch.frombuffer(bytearray(mer.swiglu_expert_header(5, 32, 32, 4096) + b"\x07" * 32), dtype=torch.uint8)
    h, payload = mer.strip_uth(t, 4096)
    assert h.dtype == 5 and payload.numel() == 32 and int(payload[0]) == 7


# -- GGUF -------------------------------------------------------------------

@pytest.mark.parametrize("version", [1, 2, 3])
@pytest.mark.parametrize("ggml,dtype", [(gs.GGML_Q4_0, 4), (gs.GGML_Q8_0, 5)])
@pytest.mark.parametrize("per_expert", [False, True])
def test_gguf_experts_byte_exact(mer, tmp_path, version, ggml, dtype, per_expert):
    """native_q4_0_interleaved_extraction_preserves_exact_bytes /
    extract_native_quant_per_expert_q4_0_passes_through: each expert's
    gate || up || down is the file's bytes, unchanged."""
    path = tmp_path / "m.gguf"
    dm, dff, ne = 64, 96, 5
    want = gs.moe_model(path, ggml, dm, dff, ne, layers=(0, 3), per_expert=per_expert, version=version, seed=version)
    with mer.GgufExperts(path) as g:
        for layer in (0, 3):
            info = g.moe_layer(layer)
            assert (info.dtype, info.d_model, info.d_ff, info.n_experts) == (dtype, dm, dff, ne)
            assert info.layout == (1 if per_expert else 0)
            assert info.expert_bytes == mer.expert_weight_bytes_for(dm, dff, mer.WeightDtype(dtype))
            for e in range(ne):
                got = g.read_expert(layer, e)
                assert got.tobytes() == b"".join(want[layer][e]), (layer, e)


def test_gguf_alignment_and_pinned_destination(mer, tmp_path):
    import torch

    path = tmp_path / "a.gguf"
    want = gs.moe_model(path, gs.GGML_Q4_0, 32, 64, 3, alignment=256)
    with mer.GgufExperts(path) as g:
        info = g.moe_layer(0)
        out = torch.zeros(info.expert_bytes + 7, dtype=torch.uint8)
        g.read_expert(0, 2, out)
        assert out[:info.expert_bytes].numpy().tobytes() == b"".join(want[0][2])
        assert not out[info.expert_bytes:].any()


def test_gguf_metadata_lookup_order(mer, tmp_path):
    """metadata_lookup (gguf_loader.rs:136-150) and
    extract_moe_prefers_expert_feed_forward_length: a dense
    feed_forward_length that disagrees with the experts is ignored when
    expert_feed_forward_length is present; the arch namespace is found
    from general.architecture."""
    path = tmp_path / "q.gguf"
    gs.moe_model(path, gs.GGML_Q8_0, 32, 64, 2, arch="qwen2moe",
                 meta={"qwen2moe.embedding_length": 32, "qwen2moe.feed_forward_length": 128,
                       "qwen2moe.expert_feed_forward_length": 64, "qwen2moe.expert_count": 2})
    with mer.GgufExperts(path) as g:
        assert g.moe_layer(0).d_ff == 64
    # only the dense key, and it disagrees: rejected
    gs.moe_model(path, gs.GGML_Q8_0, 32, 64, 2, arch="qwen2moe", meta={"qwen2moe.feed_forward_length": 128})
    with mer.GgufExperts(path) as g, pytest.raises(mer.InvalidLayout, match="feed_forward_length"):
        g.moe_layer(0)
    # llama.* wins over <arch>.*
    gs.moe_model(path, gs.GGML_Q8_0, 32, 64, 2, arch="foo",
                 meta={"llama.expert_count": 2, "foo.expert_count": 9})
    with mer.GgufExperts(path) as g:
        assert g.moe_layer(0).n_experts == 2
    # a suffix match in another namespace is used when neither is there
    gs.moe_model(path, gs.GGML_Q8_0, 32, 64, 2, arch="foo", meta={"zzz.expert_count": 3})
    with mer.GgufExperts(path) as g, pytest.raises(mer.InvalidLayout, match="expert_count"):
        g.moe_layer(0)
    # no metadata at all: geometry from the shapes
    gs.moe_model(path, gs.GGML_Q8_0, 32, 64, 2, arch="foo", meta={})
    with mer.GgufExperts(path) as g:
        assert g.moe_layer(0).n_experts == 2


@pytest.mark.parametrize("key", ["embedding_length", "expert_count"])
def test_gguf_metadata_mismatch_fails_closed(mer, tmp_path, key):
    path = tmp_path / "m.gguf"
    meta = {"mixtral.embedding_length": 32, "mixtral.expert_count": 4}
    meta[f"mixtral.{key}"] += 1
    gs.moe_model(path, gs.GGML_Q4_0, 32, 64, 4, meta=meta)
    with mer.GgufExperts(path) as g, pytest.raises(mer.InvalidLayout, match=key):
        g.read_expert(0, 0)


def test_gguf_rejects_unsupported_and_malformed(mer, tmp_path):
    path = tmp_path / "x.gguf"
    # F32 experts are not on this path
    f32 = np.zeros(32 * 64 * 2, np.float32).view(np.uint8)
    gs.write_gguf(path, [], [(f"blk.0.ffn_{p}_exps.weight", d + [2], gs.GGML_F32, f32)
                             for p, d in (("gate", [32, 64]), ("up", [32, 64]), ("down", [64, 32]))])
    with mer.GgufExperts(path) as g, pytest.raises(mer.RoutedExpertGpuIncompatibility):
        g.moe_layer(0)
    # mixed dtypes across gate / up / down
    q4 = gs.q_blocks(gs.GGML_Q4_0, 32 * 64 * 2 // 32, np.random.default_rng(0))
    q8 = gs.q_blocks(gs.GGML_Q8_0, 32 * 64 * 2 // 32, np.random.default_rng(0))
    gs.write_gguf(path, [], [("blk.0.ffn_gate_exps.weight", [32, 64, 2], gs.GGML_Q4_0, q4),
                             ("blk.0.ffn_up_exps.weight", [32, 64, 2], gs.GGML_Q4_0, q4),
                             ("blk.0.ffn_down_exps.weight", [64, 32, 2], gs.GGML_Q8_0, q8)])
    with mer.GgufExperts(path) as g, pytest.raises(mer.RoutedExpertGpuIncompatibility):
        g.moe_layer(0)
    # down shape not the transpose of gate's
    gs.write_gguf(path, [], [("blk.0.ffn_gate_exps.weight", [32, 64, 2], gs.GGML_Q4_0, q4),
                             ("blk.0.ffn_up_exps.weight", [32, 64, 2], gs.GGML_Q4_0, q4),
                             ("blk.0.ffn_down_exps.weight", [32, 64, 2], gs.GGML_Q4_0, q4)])
    with mer.GgufExperts(path) as g:
        with pytest.raises(mer.InvalidLayout, match="disagree"):
            g.moe_layer(0)
        with pytest.raises(mer.InvalidLayout, match="no expert"):
            g.moe_layer(1)
    # a layer with no experts; an expert index past the count; too small a destination
    gs.moe_model(path, gs.GGML_Q4_0, 32, 64, 2)
    with mer.GgufExperts(path) as g:
        with pytest.raises(mer.InvalidLayout, match="no expert"):
            g.moe_layer(1)
        with pytest.raises(mer.InvalidLayout, match="beyond"):
            g.read_expert(0, 2)
        with pytest.raises(mer.BufferTooSmall):
            g.read_expert(0, 0, np.empty(g.moe_layer(0).expert_bytes - 1, np.uint8))
    g.close()
    with pytest.raises(ValueError):
        g.moe_layer(0)


def test_gguf_per_expert_shape_checked(mer, tmp_path):
    path = tmp_path / "p.gguf"
    rng = np.random.default_rng(1)
    nb = 32 * 64 // 32
    t = [(f"blk.0.ffn_{p}.0.weight", [32, 64], gs.GGML_Q8_0, gs.q_blocks(gs.GGML_Q8_0, nb, rng))
         for p in ("gate", "up", "down")]  # down should be [64, 32]
    gs.write_gguf(path, [], t)
    with mer.GgufExperts(path) as g:
        assert g.moe_layer(0).n_experts == 1
        with pytest.raises(mer.InvalidLayout, match="shape"):
            g.read_expert(0, 0)


def test_gguf_file_errors(mer, tmp_path):
    with pytest.raises(OSError):
        mer.GgufExperts(tmp_path / "missing.gguf")
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + b"\0" * 60)
    with pytest.raises(mer.InvalidLayout, match="magic"):
        mer.GgufExperts(bad)
    bad.write_bytes(b"GGUF" + struct.pack("<I", 4) + b"\0" * 60)
    with pytest.raises(mer.InvalidLayout, match="version"):
        mer.GgufExperts(bad)
    # truncated header, and tensor data cut short
    path = tmp_path / "t.gguf"
    start = gs.write_gguf(path, [("general.architecture", gs.STRING, "mixtral")],
                          [("blk.0.ffn_gate_exps.weight", [32, 32, 1], gs.GGML_Q8_0, gs.q_blocks(gs.GGML_Q8_0, 32, np.random.default_rng(0))),
                           ("blk.0.ffn_up_exps.weight", [32, 32, 1], gs.GGML_Q8_0, gs.q_blocks(gs.GGML_Q8_0, 32, np.random.default_rng(1))),
                           ("blk.0.ffn_down_exps.weight", [32, 32, 1], gs.GGML_Q8_0, gs.q_blocks(gs.GGML_Q8_0, 32, np.random.default_rng(2)))])
    data = path.read_bytes()
    path.write_bytes(data[:start - 40])
    with pytest.raises(mer.InvalidLayout, match="truncated"):
        mer.GgufExperts(path)
    path.write_bytes(data[:-10])  # down's last bytes missing
    with mer.GgufExperts(path) as g, pytest.raises(mer.InvalidLayout, match="past the end"):
        g.read_expert(0, 0)
