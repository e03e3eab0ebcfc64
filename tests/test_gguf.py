"""GGUF parsing and BaseLmConfig::from_gguf through the C ABI (host only, no GPU).

Files are written by voxgen_amd.gguf; full-geometry models use a sparse data
region so the 28-layer table can be validated without 1.7 GB of disk.
"""
import ctypes as C
import struct

import numpy as np
import pytest

from voxgen_amd import abi, gguf, synth
from voxgen_amd.gguf import Gguf


def full_model(tmp_path, mutate=None, cfg_over=None, drop=None, meta_over=None, version=3):
    cfg = synth.baselm_config(context_length=32768, **(cfg_over or {}))
    m = synth.build_baselm(cfg, with_data=False)
    tensors = [t for t in m.tensors if t.name != drop]
    if mutate:
        tensors = [mutate(t) for t in tensors]
    meta = dict(m.metadata)
    meta.update(meta_over or {})
    size = max(t.offset + t.nbytes for t in tensors)
    return gguf.write(tmp_path / "m.gguf", meta, tensors, None, data_bytes=size, version=version)


def test_summary_and_tensor_table(tmp_path):
    cfg = synth.baselm_config(layers=2, hidden=256, ffn=512, vocab=64, q_heads=2, kv_heads=1)
    m = synth.build_baselm(cfg, seed=5)
    meta = dict(m.metadata)
    meta["tokenizer.ggml.tokens"] = (9, (8, ["a", "b", "c"]))
    meta["general.name"] = (8, "x" * 600)  # over 512 chars: dropped like gguf.rs:240
    p = gguf.write(tmp_path / "s.gguf", meta, m.tensors, m.data)
    g = Gguf(p)
    s = g.summary()
    assert s["version"] == 3 and s["tensor_count"] == len(m.tensors)
    assert s["metadata_count"] == len(meta) and s["alignment"] == 32
    assert s["data_offset"] % 32 == 0 and s["file_bytes"] == p.stat().st_size
    assert s["tensor_bytes"] == sum(t.nbytes for t in m.tensors)
    got = {t.name: t for t in g.tensors()}
    for t in m.tensors:
        assert got[t.name].dims == t.dims and got[t.name].offset == t.offset
        assert got[t.name].ggml_type == t.ggml_type and got[t.name].nbytes == t.nbytes
    assert g.meta("general.architecture") == "minicpm4"
    assert g.meta("minicpm4.block_count") == "2"
    with pytest.raises(abi.VxError) as e:
        g.meta("general.name")
    assert e.value.name == "VX_ERR_NOT_FOUND"
    assert g.primary_format() == abi.DTYPE_Q8_0
    # Data region bytes are where the table says.
    raw = p.read_bytes()
    t = m.tensor("blk.1.ffn_down.weight")
    a = s["data_offset"] + t.offset
    assert raw[a:a + t.nbytes] == m.data[t.offset:t.offset + t.nbytes].tobytes()


def test_config_from_full_geometry_gguf(tmp_path):
    g = Gguf(full_model(tmp_path))
    c = g.baselm_config(8192)
    assert (c["embedding_length"], c["block_count"], c["feed_forward_length"]) == (2048, 28, 6144)
    assert (c["head_count"], c["head_count_kv"], c["head_dim"], c["kv_dim"]) == (16, 2, 128, 256)
    assert c["vocab_size"] == 73448 and c["tied_output"] == 1 and c["rope_longrope"] == 1
    assert c["active_context_length"] == 8192 and c["context_length"] == 32768
    assert abs(c["rms_epsilon"] - 1e-6) < 1e-12 and c["rope_theta"] == 10000.0
    assert c["embedding_scale"] == 0.0 and c["residual_scale"] == 0.0


@pytest.mark.parametrize("case,code", [
    ("active0", "VX_ERR_INVALID_ARG"),
    ("active_big", "VX_ERR_INVALID_ARG"),
    ("layers27", "VX_ERR_UNSUPPORTED"),
    ("arch", "VX_ERR_UNSUPPORTED"),
    ("scaling", "VX_ERR_UNSUPPORTED"),
    ("missing_tensor", "VX_ERR_NOT_FOUND"),
    ("bad_dims", "VX_ERR_SHAPE"),
    ("norm_f16", "VX_ERR_SHAPE"),
    ("missing_meta", "VX_ERR_NOT_FOUND"),
])
def test_config_validation_errors(tmp_path, case, code):
    active = 8192
    kw = {}
    if case == "active0":
        active = 0
    elif case == "active_big":
        active = 40000
    elif case == "layers27":
        kw["meta_over"] = {"minicpm4.block_count": (4, 27)}
    elif case == "arch":
        kw["meta_over"] = {"general.architecture": (8, "llama")}
    elif case == "scaling":
        kw["meta_over"] = {"minicpm4.rope.scaling.type": (8, "yarn")}
    elif case == "missing_tensor":
        kw["drop"] = "blk.13.ffn_up.weight"
    elif case == "bad_dims":
        def mutate(t):
            if t.name == "blk.3.attn_k.weight":
                t = synth.TensorDesc(t.name, t.ggml_type, (2048, 512), t.offset)
            return t
        kw["mutate"] = mutate
    elif case == "norm_f16":
        def mutate(t):
            if t.name == "blk.0.attn_norm.weight":
                t = synth.TensorDesc(t.name, abi.DTYPE_F16, t.dims, t.offset)
            return t
        kw["mutate"] = mutate
    elif case == "missing_meta":
        path = full_model(tmp_path)
        m = synth.build_baselm(synth.baselm_config(context_length=32768), with_data=False)
        meta = dict(m.metadata)
        del meta["minicpm4.feed_forward_length"]
        size = max(t.offset + t.nbytes for t in m.tensors)
        path = gguf.write(tmp_path / "n.gguf", meta, m.tensors, None, data_bytes=size)
        with pytest.raises(abi.VxError) as e:
            Gguf(path).baselm_config(active)
        assert e.value.name == code
        return
    with pytest.raises(abi.VxError) as e:
        Gguf(full_model(tmp_path, **kw)).baselm_config(active)
    assert e.value.name == code


def test_head_dim_falls_back_to_rope_dimension_count(tmp_path):
    m = synth.build_baselm(synth.baselm_config(context_length=32768), with_data=False)
    meta = dict(m.metadata)
    del meta["minicpm4.attention.key_length"]
    size = max(t.offset + t.nbytes for t in m.tensors)
    p = gguf.write(tmp_path / "k.gguf", meta, m.tensors, None, data_bytes=size)
    assert Gguf(p).baselm_config(4096)["head_dim"] == 128


def test_rope_original_context_and_long_factor_scaling(tmp_path):
    p = full_model(tmp_path, meta_over={"minicpm4.rope.scaling.original_context_length": (4, 4096)})
    c = Gguf(p).baselm_config(8192)
    assert c["rope_original_context_length"] == 4096


@pytest.mark.parametrize("how", ["magic", "version1", "version4", "truncated_header", "tensor_past_eof",
                                 "bad_type", "rank0", "q8_not_div32", "f32_size_overflow",
                                 "q8_size_overflow", "offset_overflow"])
def test_parse_errors(tmp_path, how):
    cfg = synth.baselm_config(layers=1, hidden=256, ffn=512, vocab=64, q_heads=2, kv_heads=1)
    m = synth.build_baselm(cfg, seed=1)
    tensors, data, version = list(m.tensors), m.data, 3
    if how == "version1":
        version = 1
    if how == "version4":
        version = 4
    if how == "bad_type":
        tensors[0] = synth.TensorDesc(tensors[0].name, 2, tensors[0].dims, tensors[0].offset, 64)
    if how == "rank0":
        tensors[1] = synth.TensorDesc(tensors[1].name, 0, (), tensors[1].offset, 4)
    if how == "q8_not_div32":
        t = tensors[-1]
        tensors[-1] = synth.TensorDesc(t.name, 8, (40, 2), t.offset, 102)
    # Sizes that wrap 64 bits (gguf.rs:37-48 checked_mul): 2^62 f32 elements are
    # 2^64 bytes, and 1024 x 16954728008924221 Q8_0 weights are 34/32 of a count
    # that fits 64 bits but whose byte size does not.
    if how == "f32_size_overflow":
        t = tensors[-1]
        tensors[-1] = synth.TensorDesc(t.name, 0, (1 << 62, 1), t.offset, 1)
    if how == "q8_size_overflow":
        t = tensors[-1]
        tensors[-1] = synth.TensorDesc(t.name, 8, (1024, 16954728008924221), t.offset, 1)
    # data_offset + offset + bytes wraps (gguf.rs:281 checked_add).
    if how == "offset_overflow":
        t = tensors[-1]
        tensors[-1] = synth.TensorDesc(t.name, t.ggml_type, t.dims, (1 << 64) - 64, t.nbytes)
    p = gguf.write(tmp_path / "e.gguf", m.metadata, tensors, data, version=version)
    raw = bytearray(p.read_bytes())
    if how == "magic":
        raw[0:4] = b"GGUX"
    if how == "truncated_header":
        raw = raw[:40]
    if how == "tensor_past_eof":
        raw = raw[:-4096]
    p.write_bytes(bytes(raw))
    with pytest.raises(abi.VxError) as e:
        Gguf(p)
    assert e.value.name == "VX_ERR_GGUF"


def test_writer_layout_is_gguf_v3():
    hdr = gguf.header_bytes({"a": (4, 7)}, [synth.TensorDesc("t", 0, (3,), 0)])
    magic, ver, nt, nm = struct.unpack_from("<IIQQ", hdr)
    assert (magic, ver, nt, nm) == (0x46554747, 3, 1, 1)
    assert len(hdr) % 32 == 0


# ----------------------------------------------- AcousticConfig::from_gguf
def acoustic_file(tmp_path, mutate=None, drop=None, meta_over=None):
    acfg = synth.acoustic_config()
    m = synth.build_acoustic(acfg, with_data=False)
    tensors = [t for t in m.tensors if t.name != drop]
    if mutate:
        tensors = [mutate(t) for t in tensors]
    meta = dict(m.metadata)
    meta.update(meta_over or {})
    size = max(t.offset + t.nbytes for t in tensors)
    return gguf.write(tmp_path / "a.gguf", meta, tensors, None, data_bytes=size)


def test_acoustic_config_from_gguf(tmp_path):
    base = synth.baselm_config(context_length=32768, residual_scale=0.0)
    c = Gguf(acoustic_file(tmp_path)).acoustic_config(base, 4096)
    want = synth.acoustic_config(active_context=4096)
    for k, v in want.items():
        assert c[k] == pytest.approx(v), k
    base["residual_scale"] = 0.25
    assert Gguf(acoustic_file(tmp_path)).acoustic_config(base, 1)["residual_scale"] == 0.25


def _retype(name, ty):
    def mutate(t):
        return synth.TensorDesc(t.name, ty, t.dims, t.offset) if t.name == name else t
    return mutate


@pytest.mark.parametrize("case,code", [
    ("arch", "VX_ERR_UNSUPPORTED"), ("version", "VX_ERR_UNSUPPORTED"), ("ctx0", "VX_ERR_INVALID_ARG"),
    ("ctx_big", "VX_ERR_INVALID_ARG"), ("layers7", "VX_ERR_UNSUPPORTED"), ("rope", "VX_ERR_UNSUPPORTED"),
    ("bool", "VX_ERR_GGUF"), ("scale0", "VX_ERR_INVALID_ARG"), ("base", "VX_ERR_UNSUPPORTED"),
    ("missing", "VX_ERR_NOT_FOUND"), ("fsq_bias_f32", "VX_ERR_SHAPE"), ("q8", "VX_ERR_UNSUPPORTED"),
    ("norm_f16", "VX_ERR_SHAPE"), ("stop_dims", "VX_ERR_SHAPE"), ("missing_meta", "VX_ERR_NOT_FOUND"),
])
def test_acoustic_config_errors(tmp_path, case, code):
    base = synth.baselm_config(context_length=32768)
    active, kw = 512, {}
    if case == "arch":
        kw["meta_over"] = {"general.architecture": (8, "minicpm4")}
    elif case == "version":
        kw["meta_over"] = {"voxcpm.model_version": (6, 1.5)}
    elif case == "ctx0":
        active = 0
    elif case == "ctx_big":
        active = 8193
    elif case == "layers7":
        kw["meta_over"] = {"voxcpm.residual_lm.n_layer": (4, 7)}
    elif case == "rope":
        kw["meta_over"] = {"voxcpm.residual_lm.no_rope": (7, False)}
    elif case == "bool":
        kw["meta_over"] = {"voxcpm.residual_lm.no_rope": (8, "yes")}
    elif case == "scale0":
        kw["meta_over"] = {"voxcpm.fsq.scale": (6, 0.0)}
    elif case == "base":
        base["feed_forward_length"] = 4096
    elif case == "missing":
        kw["drop"] = "residual_lm.blk.5.ffn_down.weight"
    elif case == "fsq_bias_f32":   # require_vector(.., allow_f32 = false)
        kw["mutate"] = _retype("fsq.in_proj.bias", abi.DTYPE_F32)
    elif case == "q8":             # validate_acoustic_f16
        kw["mutate"] = _retype("residual_lm.blk.0.attn_q.weight", abi.DTYPE_Q8_0)
    elif case == "norm_f16":
        kw["mutate"] = _retype("residual_lm.blk.2.ffn_norm.weight", abi.DTYPE_F16)
    elif case == "stop_dims":
        def mutate(t):
            if t.name == "stop_predictor.linear2.weight":
                t = synth.TensorDesc(t.name, t.ggml_type, (2048, 3), t.offset)
            return t
        kw["mutate"] = mutate
    elif case == "missing_meta":
        acfg = synth.acoustic_config()
        m = synth.build_acoustic(acfg, with_data=False)
        meta = dict(m.metadata)
        del meta["voxcpm.fsq.latent_dim"]
        size = max(t.offset + t.nbytes for t in m.tensors)
        path = gguf.write(tmp_path / "b.gguf", meta, m.tensors, None, data_bytes=size)
        with pytest.raises(abi.VxError) as e:
            Gguf(path).acoustic_config(base, active)
        assert e.value.name == code
        return
    with pytest.raises(abi.VxError) as e:
        Gguf(acoustic_file(tmp_path, **kw)).acoustic_config(base, active)
    assert e.value.name == code


# --------------------------------------------- AudioVaeConfig::from_gguf
def vae_file(tmp_path, mutate=None, drop=None, meta_over=None):
    cfg = synth.audiovae_config()
    m = synth.build_audiovae(cfg, encoder=True, with_data=False)
    tensors = [t for t in m.tensors if t.name != drop]
    if mutate:
        tensors = [mutate(t) for t in tensors]
    meta = dict(m.metadata)
    meta.update(meta_over or {})
    size = max(t.offset + t.nbytes for t in tensors)
    return gguf.write(tmp_path / "v.gguf", meta, tensors, None, data_bytes=size)


def test_audiovae_config_from_gguf(tmp_path):
    c = Gguf(vae_file(tmp_path)).audiovae_config()
    want = synth.audiovae_config()
    for k, v in want.items():
        assert c[k] == v, k
    assert c["decoder_hop"] == 1920 and c["encoder_hop"] == 640 and c["decoder_sr_bucket"] == 3


@pytest.mark.parametrize("case,code", [
    ("version", "VX_ERR_UNSUPPORTED"), ("dec", "VX_ERR_UNSUPPORTED"), ("cond", "VX_ERR_UNSUPPORTED"),
    ("missing_enc", "VX_ERR_NOT_FOUND"), ("missing_dec", "VX_ERR_NOT_FOUND"), ("f32_alpha", "VX_ERR_SHAPE"),
    ("convt_dims", "VX_ERR_SHAPE"), ("embed_dims", "VX_ERR_SHAPE"), ("no_meta", "VX_ERR_NOT_FOUND"),
])
def test_audiovae_config_errors(tmp_path, case, code):
    kw = {}
    if case == "version":
        kw["meta_over"] = {"voxcpm.model_version": (6, 1.0)}
    elif case == "dec":
        kw["meta_over"] = {"voxcpm.audiovae.decoder_dim": (4, 1024)}
    elif case == "cond":
        kw["meta_over"] = {"voxcpm.audiovae.cond_type": (8, "film")}
    elif case == "missing_enc":
        kw["drop"] = "audio_vae.encoder.fc_logvar"
    elif case == "missing_dec":
        kw["drop"] = "audio_vae.decoder.model.5.block.3.block.2.alpha"
    elif case == "f32_alpha":
        kw["mutate"] = _retype("audio_vae.decoder.model.8.alpha", abi.DTYPE_F32)
    elif case == "convt_dims":
        def mutate(t):
            if t.name == "audio_vae.decoder.model.3.block.1":
                t = synth.TensorDesc(t.name, t.ggml_type, (12, 1024, 512), t.offset)
            return t
        kw["mutate"] = mutate
    elif case == "embed_dims":
        def mutate(t):
            if t.name == "audio_vae.decoder.sr_cond_model.4.bias_embed":
                t = synth.TensorDesc(t.name, t.ggml_type, (512, 3), t.offset)
            return t
        kw["mutate"] = mutate
    elif case == "no_meta":
        kw["meta_over"] = {}
        cfg = synth.audiovae_config()
        m = synth.build_audiovae(cfg, encoder=True, with_data=False)
        meta = dict(m.metadata)
        del meta["voxcpm.audiovae.out_sample_rate"]
        size = max(t.offset + t.nbytes for t in m.tensors)
        path = gguf.write(tmp_path / "w.gguf", meta, m.tensors, None, data_bytes=size)
        with pytest.raises(abi.VxError) as e:
            Gguf(path).audiovae_config()
        assert e.value.name == code
        return
    with pytest.raises(abi.VxError) as e:
        Gguf(vae_file(tmp_path, **kw)).audiovae_config()
    assert e.value.name == code


@pytest.mark.parametrize("dims,ty,code", [
    ((1 << 62, 1), 0, "VX_ERR_GGUF"),                   # f32 byte size wraps
    ((1024, 16954728008924221), 8, "VX_ERR_GGUF"),      # Q8_0 byte size wraps
    ((1 << 33, 1 << 32), 1, "VX_ERR_GGUF"),             # element count wraps
])
def test_model_upload_refuses_overflowing_tables_before_device_work(dims, ty, code):
    """The upload validates its tensor table with checked arithmetic before it uses
    the context, so these tables are refused here without a GPU (a null context)."""
    data = np.zeros(4096, dtype=np.uint8)
    arr = (abi.TensorInfo * 1)(synth.TensorDesc("w", ty, dims, 0, 1).to_c())
    h = abi.MODEL()
    with pytest.raises(abi.VxError) as e:
        abi.call("vx_model_upload", None, data.ctypes.data_as(C.c_void_p), data.nbytes, arr, 1, C.byref(h))
    assert e.value.name == code


# ------------------------------------- parse rules shared with gguf.rs / baselm.rs
def test_invalid_utf8_string_is_refused(tmp_path):
    """gguf.rs:182 reads strings with std::str::from_utf8: a metadata key or value
    that is not UTF-8 fails the load."""
    p = full_model(tmp_path)
    raw = bytearray(p.read_bytes())
    i = raw.find(b"general.architecture")
    assert i > 0
    raw[i + 3] = 0xFF  # a lone continuation-less byte
    p.write_bytes(bytes(raw))
    with pytest.raises(abi.VxError) as e:
        Gguf(p)
    assert e.value.name == "VX_ERR_GGUF"


def test_rank_up_to_8_is_accepted(tmp_path):
    """gguf.rs:253-256 accepts n_dims <= 8; an unused rank-6 tensor does not stop
    the model from loading, and is listed with its upper dims folded into dims[3]."""
    extra = synth.TensorDesc("unused.rank6", 0, (2, 3, 4, 5, 6, 7), 0)
    cfg = synth.baselm_config(context_length=32768)
    m = synth.build_baselm(cfg, with_data=False)
    tensors = list(m.tensors) + [extra]
    size = max(t.offset + t.nbytes for t in tensors)
    p = gguf.write(tmp_path / "r.gguf", m.metadata, tensors, None, data_bytes=size)
    g = Gguf(p)
    t = {x.name: x for x in g.tensors()}["unused.rank6"]
    assert t.dims == (2, 3, 4, 5 * 6 * 7)
    assert g.baselm_config(4096)["block_count"] == 28


def test_zero_element_tensor_with_large_upper_dims_is_accepted(tmp_path):
    """gguf.rs's checked element product is 0 once a dim is 0, so a tensor with a
    zero dim loads whatever its other dims; folding dims 5..8 of such a tensor
    into dims[3] must not fail on an overflow the element count never has."""
    big = 1 << 40
    extra = synth.TensorDesc("unused.empty", 0, (0, 3, 4, big, big, 7), 0)
    cfg = synth.baselm_config(context_length=32768)
    m = synth.build_baselm(cfg, with_data=False)
    tensors = list(m.tensors) + [extra]
    size = max(t.offset + t.nbytes for t in tensors)
    p = gguf.write(tmp_path / "z.gguf", m.metadata, tensors, None, data_bytes=size)
    g = Gguf(p)
    t = {x.name: x for x in g.tensors()}["unused.empty"]
    assert t.dims[:3] == (0, 3, 4) and t.dims[3] == 0 and t.nbytes == 0
    assert g.baselm_config(4096)["block_count"] == 28


@pytest.mark.parametrize("text,ok", [("28", True), ("+28", True), (" 28", False), ("28 ", False),
                                     ("0x1c", False), ("-28", False), ("2.8e1", False), ("", False)])
def test_string_metadata_parses_like_rust_u32(tmp_path, text, ok):
    """baselm.rs:275 parses metadata text with str::parse::<u32>: digits with an
    optional '+', nothing else. A value that does not parse counts as missing."""
    p = full_model(tmp_path, meta_over={"minicpm4.block_count": (8, text)})
    if ok:
        assert Gguf(p).baselm_config(4096)["block_count"] == 28
    else:
        with pytest.raises(abi.VxError) as e:
            Gguf(p).baselm_config(4096)
        assert e.value.name == "VX_ERR_NOT_FOUND"  # "missing required metadata"


@pytest.mark.parametrize("text,want", [("1e-6", 1e-6), ("+1e-6", 1e-6), ("0.000001", 1e-6),
                                       (" 1e-6", None), ("0x1p-20", None), ("1e-6\n", None)])
def test_string_metadata_parses_like_rust_f32(tmp_path, text, want):
    """baselm.rs:281 parses metadata text with str::parse::<f32>: no surrounding
    whitespace and no hexadecimal floats (which strtof alone would accept)."""
    p = full_model(tmp_path, meta_over={"minicpm4.attention.layer_norm_rms_epsilon": (8, text)})
    if want is not None:
        assert Gguf(p).baselm_config(4096)["rms_epsilon"] == pytest.approx(want)
    else:
        with pytest.raises(abi.VxError) as e:
            Gguf(p).baselm_config(4096)
        assert e.value.name == "VX_ERR_NOT_FOUND"  # "missing required metadata"
