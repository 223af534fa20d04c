"""CPU: the GGUF reader of libdmoe (dmoe_gguf_*, the loader mechanics of
src/diffuse-model.cpp:5-73,143-198 for the MoE tensors).

Pinned three ways: a known-answer file assembled byte by byte here from the
container layout (not by the test writer), a round trip through the writer in
tests/gguf_writer.py with every tensor compared byte for byte, and malformed
files (every truncation of a small file, bad magic / version / alignment,
data past the end) that must be refused without reading past the mapping."""
import ctypes as C
import struct

import numpy as np
import pytest

from gguf_writer import (ARR, F32, GGUFWriter, I32, STR, U32, U8, add_attn_layer, add_dense_layer, add_moe_layer,
                         attn_keys, moe_keys)


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _kat_bytes():
    """GGUF v3: 5 key/values (u32, f32, string, array of u8, i64), two tensors
    (F32 [4] at offset 0, F16 [8, 2] at offset 32), alignment 32."""
    kv = [
        _s("diffuse.expert_count") + struct.pack("<II", 4, 16),
        _s("qwen2.routed_scaling_factor") + struct.pack("<If", 6, 2.5),
        _s("general.name") + struct.pack("<I", 8) + _s("kat"),
        _s("general.blob") + struct.pack("<IIQ", 9, 0, 3) + bytes([7, 8, 9]),
        _s("llama.expert_capacity") + struct.pack("<Iq", 11, 12),
    ]
    ti = [
        _s("a.weight") + struct.pack("<IQIQ", 1, 4, 0, 0),
        _s("b.weight") + struct.pack("<IQQIQ", 2, 8, 2, 1, 32),
    ]
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, len(kv)) + b"".join(kv) + b"".join(ti)
    head += b"\0" * ((-len(head)) % 32)
    a = np.array([1.0, -2.0, 3.5, 0.25], np.float32).tobytes()
    b = np.arange(16, dtype=np.float16).tobytes()
    return head + a + b"\0" * (32 - len(a)) + b, len(head)


def test_known_answer_file(tmp_path):
    from dmoe.gguf import GGUF
    raw, data_start = _kat_bytes()
    p = tmp_path / "kat.gguf"
    p.write_bytes(raw)
    with GGUF(p) as g:
        assert g.get_u32("expert_count") == 16                     # diffuse. prefix
        assert g.get_f32("routed_scaling_factor") == 2.5            # qwen2. prefix
        assert g.get_u32("expert_capacity") == 12                   # llama. prefix, an i64 value
        assert g.get_u32("expert_used_count") is None
        assert g.tensor_names() == ["a.weight", "b.weight"]
        a = g.tensor("a.weight")
        assert (a.type, list(a.ne), list(a.nb)) == (0, [4, 1, 1, 1], [4, 16, 16, 16])
        assert C.string_at(a.data, 16) == raw[data_start:data_start + 16]
        b = g.tensor("b.weight")
        assert (b.type, list(b.ne), list(b.nb)) == (1, [8, 2, 1, 1], [2, 16, 32, 32])
        assert np.array_equal(np.frombuffer(C.string_at(b.data, 32), np.float16), np.arange(16))


def _tiny_file(tmp_path, O, prefix="diffuse"):
    from dmoe import synth
    cfg = synth.CONFIGS["tiny"]
    w = synth.host_layer(cfg, 3, O.quantize_rows)
    d = synth.host_dense(256, 512, 12, 4, O.quantize_rows)
    wr = GGUFWriter()
    for k, t, v in moe_keys(w, n_layer=2, first_k_dense=1, prefix=prefix):
        wr.add(k, t, v)
    wr.add("general.architecture", STR, prefix)
    wr.add("tokenizer.ggml.tokens", ARR, (STR, ["a", "bb", "ccc"]))
    add_dense_layer(wr, 0, d)
    add_moe_layer(wr, 1, w)
    p = tmp_path / "tiny.gguf"
    wr.write(p)
    return p, w, d


@pytest.mark.parametrize("prefix", ["diffuse", "qwen2", "llama"])
def test_round_trip_tiny_layer(tmp_path, O, prefix):
    from dmoe.gguf import GGUF
    p, w, d = _tiny_file(tmp_path, O, prefix)
    with GGUF(p) as g:
        hp, n_layer, fk = g.moe_hparams()
        assert (n_layer, fk) == (2, 1)
        ref = w.hparams()
        for f in ("n_embd", "n_experts", "top_k", "capacity", "block_size", "moe_ff", "n_shared",
                  "shared_ff", "norm_topk_prob"):
            assert getattr(hp, f) == getattr(ref, f), f
        assert hp.routed_scaling == np.float32(2.5)
        lw = g.layer_weights(1)
        for f in ("gate_w", "gate_bias", "exp_gate", "exp_up", "exp_down", "sh_gate", "sh_up", "sh_down"):
            assert np.array_equal(np.asarray(getattr(lw, f)).view(np.uint8).reshape(-1),
                                  np.asarray(getattr(w, f)).view(np.uint8).reshape(-1)), f
        # the oracle on the mapped tensors equals the oracle on the originals
        x = np.random.default_rng(0).standard_normal((32, 256)).astype(np.float32)
        assert np.array_equal(O.layer_forward(lw, x), O.layer_forward(w, x))
        dw = g.dense_weights(0)
        assert (dw.n_embd, dw.n_ff, dw.wtype) == (256, 512, 12)
        for f in ("gate", "up", "down"):
            assert np.array_equal(getattr(dw, f), getattr(d, f)), f
        desc = g.layer_desc(1)
        assert desc.exp_gate.nb[1] == 256 * 4 and desc.exp_gate.nb[2] == 256 * 4 * 128


def test_defaults_and_missing(tmp_path):
    """Missing optional keys take the reference's defaults (capacity 48,
    moe_block_size = block_length or 32, norm_topk_prob 1, routed_scaling 1);
    a missing required key or tensor is DMOE_ERR_NOT_FOUND."""
    import dmoe
    from dmoe.gguf import GGUF
    wr = GGUFWriter()
    wr.add("diffuse.block_count", U32, 1)
    wr.add("diffuse.embedding_length", U32, 256)
    wr.add("diffuse.block_length", U32, 64)
    p = tmp_path / "d.gguf"
    wr.write(p)
    with GGUF(p) as g:
        hp, nl, fk = g.moe_hparams()
        assert (hp.capacity, hp.block_size, hp.norm_topk_prob, hp.routed_scaling, nl, fk) == (48, 64, 1, 1.0, 1, 0)
        with pytest.raises(dmoe.DmoeError) as ei:
            g.layer_desc(0)
        assert ei.value.code == dmoe._abi.ERR_NOT_FOUND
    wr = GGUFWriter()
    wr.add("diffuse.block_count", U32, 1)
    wr.write(p)
    with GGUF(p) as g:
        with pytest.raises(dmoe.DmoeError) as ei:
            g.moe_hparams()                                       # embedding_length missing
        assert ei.value.code == dmoe._abi.ERR_NOT_FOUND


@pytest.mark.parametrize("qk_norm", [True, False])
def test_attention_round_trip(tmp_path, O, qk_norm):
    """The attention keys and blk.N.attn_* tensors written by the converter's
    layout come back as the AttnWeights they were written from; the oracle
    on the mapped tensors equals the oracle on the originals."""
    from dmoe import synth
    from dmoe.gguf import GGUF
    a = synth.host_attn(12, 3, O.quantize_rows, 256, 4, 2, 64, 32, block_length=16, rope_base=5e5,
                        rms_eps=1e-5, qk_norm=qk_norm)
    wr = GGUFWriter()
    wr.add("diffuse.block_count", U32, 2)
    wr.add("diffuse.embedding_length", U32, 256)
    for k, t, v in attn_keys(a):
        wr.add(k, t, v)
    add_attn_layer(wr, 1, a)
    p = tmp_path / "attn.gguf"
    wr.write(p)
    with GGUF(p) as g:
        ap = g.attn_hparams()
        assert (ap.n_embd, ap.n_head, ap.n_head_kv, ap.head_dim, ap.rotary_dim, ap.use_qk_norm,
                ap.block_length) == (256, 4, 2, 64, 32, int(qk_norm), 16)
        assert ap.rope_base == np.float32(5e5) and ap.rms_eps == np.float32(1e-5)
        aw = g.attn_weights(1)
        for f in ("attn_norm", "qkv", "wo", "post_norm", "q_norm", "k_norm"):
            x, y = getattr(aw, f), getattr(a, f)
            if y is None:
                assert x is None, f
            else:
                assert np.array_equal(np.asarray(x).view(np.uint8).reshape(-1),
                                      np.asarray(y).view(np.uint8).reshape(-1)), f
        h = synth.normal(4, 1, 24 * 256).reshape(24, 256)
        r0, r1 = O.attn_forward(aw, h), O.attn_forward(a, h)
        assert np.array_equal(r0[0], r1[0]) and np.array_equal(r0[1], r1[1])
        import dmoe
        with pytest.raises(dmoe.DmoeError) as ei:
            g.attn_desc(0, qk_norm)                             # layer 0 has no attention tensors
        assert ei.value.code == dmoe._abi.ERR_NOT_FOUND


def test_attention_defaults(tmp_path):
    """head_dim = n_embd / n_head, rotary_dim = head_dim, no QK norm, block
    length 0, rope base 1e6, eps 1e-6 when the keys are absent; head counts
    are required."""
    import dmoe
    from dmoe.gguf import GGUF
    wr = GGUFWriter()
    wr.add("llama.embedding_length", U32, 512)
    wr.add("llama.attention.head_count", U32, 8)
    wr.add("llama.attention.head_count_kv", U32, 2)
    p = tmp_path / "a.gguf"
    wr.write(p)
    with GGUF(p) as g:
        ap = g.attn_hparams()
        assert (ap.head_dim, ap.rotary_dim, ap.use_qk_norm, ap.block_length) == (64, 64, 0, 0)
        assert ap.rope_base == np.float32(1e6) and ap.rms_eps == np.float32(1e-6)
    wr = GGUFWriter()
    wr.add("diffuse.embedding_length", U32, 512)
    wr.add("diffuse.attention.head_count", U32, 8)
    wr.write(p)
    with GGUF(p) as g:
        with pytest.raises(dmoe.DmoeError) as ei:
            g.attn_hparams()                                      # head_count_kv missing
        assert ei.value.code == dmoe._abi.ERR_NOT_FOUND


def test_malformed_files_are_refused(tmp_path):
    import dmoe
    from dmoe.gguf import GGUF
    raw, _ = _kat_bytes()
    p = tmp_path / "m.gguf"

    def code(data):
        p.write_bytes(data)
        try:
            GGUF(p).close()
            return 0
        except dmoe.DmoeError as e:
            return e.code

    assert code(raw) == 0
    # every truncation: refused (the last tensor's data runs past the end), never a crash
    for n in range(len(raw)):
        assert code(raw[:n]) == dmoe._abi.ERR_FORMAT, n
    assert code(b"GGUX" + raw[4:]) == dmoe._abi.ERR_FORMAT                       # magic
    assert code(raw[:4] + struct.pack("<I", 9) + raw[8:]) == dmoe._abi.ERR_FORMAT  # version
    huge = raw[:8] + struct.pack("<Q", 1 << 40) + raw[16:]                        # tensor count
    assert code(huge) == dmoe._abi.ERR_FORMAT
    wr = GGUFWriter()
    wr.add("general.alignment", U32, 24)                                         # not a power of two
    wr.write(p)
    with pytest.raises(dmoe.DmoeError) as ei:
        GGUF(p)
    assert ei.value.code == dmoe._abi.ERR_FORMAT
    with pytest.raises(dmoe.DmoeError) as ei:
        GGUF(tmp_path / "absent.gguf")
    assert ei.value.code == dmoe._abi.ERR_NOT_FOUND


def test_alignment_key_and_u8_values(tmp_path):
    from dmoe.gguf import GGUF
    wr = GGUFWriter(alignment=64)
    wr.add("general.alignment", U32, 64)
    wr.add("diffuse.expert_count", U8, 200)
    wr.add_tensor("t.weight", 0, [3], np.array([1, 2, 3], np.float32))
    wr.add_tensor("u.weight", 0, [2], np.array([4, 5], np.float32))
    p = tmp_path / "a.gguf"
    wr.write(p)
    with GGUF(p) as g:
        assert g.get_u32("expert_count") == 200
        t, u = g.tensor("t.weight"), g.tensor("u.weight")
        assert t.data % 64 == 0 and u.data - t.data == 64
        assert np.frombuffer(C.string_at(u.data, 8), np.float32).tolist() == [4.0, 5.0]


def test_views_keep_the_mapping(tmp_path, O):
    """The arrays layer_weights / dense_weights return stay readable after the
    GGUF object is closed or dropped: each view holds the mapping."""
    import gc
    from dmoe.gguf import GGUF
    p, w, d = _tiny_file(tmp_path, O)
    lw = GGUF(p).layer_weights(1)            # the handle object is dropped at once
    gc.collect()
    assert np.array_equal(lw.exp_down.reshape(-1), np.asarray(w.exp_down).view(np.uint8).reshape(-1))
    g = GGUF(p)
    dw = g.dense_weights(0)
    g.close()
    del g
    gc.collect()
    assert np.array_equal(dw.down, d.down)
    with GGUF(p) as g2:
        gw = g2.layer_weights(1).gate_w
    assert np.array_equal(gw, w.gate_w)
    import dmoe
    with pytest.raises(dmoe.DmoeError):
        g2.layer_desc(1)                     # the object itself is closed


def _mismatch_file(tmp_path, O, key, value, vtype=U32):
    from dmoe import synth
    cfg = synth.CONFIGS["tiny"]
    w = synth.host_layer(cfg, 3, O.quantize_rows)
    wr = GGUFWriter()
    for k, t, v in moe_keys(w, n_layer=1):
        if k == f"diffuse.{key}":
            t, v = vtype, value
        wr.add(k, t, v)
    add_moe_layer(wr, 0, w)
    p = tmp_path / f"mm_{key}.gguf"
    wr.write(p)
    return p


@pytest.mark.parametrize("key,value", [("expert_count", 64), ("expert_feed_forward_length", 256),
                                       ("embedding_length", 512)])
def test_tensor_shape_against_hparams(tmp_path, O, key, value):
    """Hyper-parameters that disagree with a tensor's own ne (64 experts in
    the metadata, 16 in the tensors) are refused with DMOE_ERR_SHAPE instead
    of a view sized from the metadata, which would reach past the tensor."""
    import dmoe
    from dmoe.gguf import GGUF
    p = _mismatch_file(tmp_path, O, key, value)
    with GGUF(p) as g:
        with pytest.raises(dmoe.DmoeError) as ei:
            g.layer_weights(0)
        assert ei.value.code == dmoe._abi.ERR_SHAPE


@pytest.mark.parametrize("vtype,value", [(F32, 16.0), (I32, -4), (STR, "16")])
def test_optional_key_of_wrong_type(tmp_path, O, vtype, value):
    """An optional key that is present but not a non-negative integer (an f32
    expert_count, a negative one, a string) is DMOE_ERR_FORMAT, as a type
    mismatch is for gguf_get_val_u32, not the default."""
    import dmoe
    from dmoe.gguf import GGUF
    p = _mismatch_file(tmp_path, O, "expert_count", value, vtype)
    with GGUF(p) as g:
        with pytest.raises(dmoe.DmoeError) as ei:
            g.moe_hparams()
        assert ei.value.code == dmoe._abi.ERR_FORMAT


@pytest.mark.parametrize("tied", [False, True])
def test_head_weights(tmp_path, O, tied):
    """output_norm.weight and output.weight (Q6_K, as the reference's Q4_K
    schemes write it) read back as a HeadWeights of views; without
    output.weight the tied token_embd.weight (F16) is the LM head, as the
    reference's loader falls back (src/diffuse-model.cpp:137-138)."""
    from dmoe.gguf import GGUF
    rng = np.random.default_rng(5)
    H, V = 512, 96
    norm = rng.uniform(0.5, 1.5, H).astype(np.float32)
    f = (rng.standard_normal((V, H)) * 0.02).astype(np.float32)
    wr = GGUFWriter()
    wr.add("diffuse.embedding_length", U32, H)
    wr.add_tensor("output_norm.weight", 0, [H], norm)
    if tied:
        out, t = f.astype(np.float16).view(np.uint8).reshape(V, -1), 1
        wr.add_tensor("token_embd.weight", 1, [H, V], out)
    else:
        out, t = O.quantize_rows(14, f), 14
        wr.add_tensor("output.weight", 14, [H, V], out)
    p = tmp_path / "h.gguf"
    wr.write(p)
    with GGUF(p) as g:
        hw = g.head_weights()
    assert (hw.n_embd, hw.n_vocab, hw.wtype) == (H, V, t)
    assert np.array_equal(hw.norm, norm)
    assert np.array_equal(hw.output, out)
    assert hw.output.shape == (V, 210 * H // 256 if t == 14 else 2 * H)
