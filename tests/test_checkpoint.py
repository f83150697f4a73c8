"""The reference's ActorCritic checkpoint formats (save_ppo_model / load_ppo_model,
src/main.rs:123-166) through the library's C ABI. Host functions only: these run without a GPU.

There is no checkpoint file in the reference repository and the Rust crate cannot be built here,
so the formats are pinned by an independent encoder written below from the published serde data
model and bincode 1.3's fixed-width encoding, and by the struct declarations of the reference
(field names and order: src/ppo.rs:246-251, src/transformer.rs:8-17, 35-45, 219-225, 374-398,
src/nn.rs:11-17, 144-149, src/autograd.rs:22-49). Byte-level parity with the real serde_json text
is unpinned: the JSON is checked as a document (keys, order, values), which is what the
reference's reader consumes.
"""
import ctypes
import json
import math
import os
import struct

import numpy as np
import pytest

import talos_hip as th
import workload


def cfg(B=4, S=16, **over):
    a = list(workload.REFERENCE_ACTOR_CRITIC)
    c = th.PpoCfg(B, S, *a)
    for k, v in over.items():
        setattr(c, k, v)
    return c


def params_for(c, seed=0):
    return workload.ppo_params(np.random.default_rng(seed), c).astype(np.float32)


# ---------------------------------------------------------------------------
# An independent serde tree of ActorCritic, written from the Rust declarations
# ---------------------------------------------------------------------------
def _tree(c, p, max_seq_len=256, base=10000.0, eps=1e-5):
    """(kind, value) nodes: ("struct", [(name, node)]), ("vecf", [...]), ("vecu", [...]),
    ("u", int), ("f", float), ("opt", node | None). p: float64 values in layout order."""
    it = iter(np.asarray(p, np.float64).tolist())

    def tensor(*shape):
        n = int(np.prod(shape))
        return ("struct", [("data", ("vecf", [next(it) for _ in range(n)])), ("shape", ("vecu", list(shape)))])

    def linear(fin, fout, bias):
        w = tensor(fin, fout)
        b = tensor(fout) if bias else None
        return ("struct", [("weight", w), ("bias", ("opt", b)), ("in_features", ("u", fin)),
                           ("out_features", ("u", fout))])

    def rms(d):
        return ("struct", [("weight", tensor(d)), ("eps", ("f", eps)), ("dim", ("u", d))])

    d, H, L, r, vd, F, A, I = c.d_model, c.n_heads, c.kv_latent, c.rope_dim, c.v_dim, c.ffn_dim, c.n_actions, c.in_dim
    cos, sin = [], []
    for pos in range(max_seq_len):  # RoPE::precompute, src/transformer.rs:239-251
        for i in range(r // 2):
            theta = 1.0 / math.pow(base, (2 * i) / r)
            cos.append(math.cos(pos * theta))
            sin.append(math.sin(pos * theta))
    embed = linear(I, d, True)
    n1 = rms(d)
    mla = ("struct", [
        ("config", ("struct", [("dim", ("u", d)), ("num_heads", ("u", H)), ("q_lora_rank", ("u", 0)),
                               ("kv_lora_rank", ("u", L)), ("qk_rope_dim", ("u", r)), ("v_head_dim", ("u", vd)),
                               ("max_seq_len", ("u", max_seq_len))])),
        ("w_dkv", linear(d, L, False)), ("w_uk", linear(L, H * vd, False)), ("w_uv", linear(L, H * vd, False)),
        ("w_q", linear(d, H * vd, False)), ("w_kr", linear(d, H * r, False)), ("w_qr", linear(d, H * r, False)),
        ("w_o", linear(H * vd, d, False)),
        ("rope", ("struct", [("dim", ("u", r)), ("base", ("f", base)), ("cos_cache", ("vecf", cos)),
                             ("sin_cache", ("vecf", sin))]))])
    n2 = rms(d)
    f1, f2 = linear(d, F, True), linear(F, d, True)
    nf = rms(d)
    out = linear(d, d, True)
    backbone = ("struct", [("embed", embed), ("norm_1", n1), ("mla_layer", mla), ("norm_2", n2), ("ffn_1", f1),
                           ("ffn_2", f2), ("norm_final", nf), ("out_proj", out)])
    root = ("struct", [("backbone", backbone), ("actor_head", linear(d, A, True)),
                       ("critic_head", linear(d, 1, True))])
    assert next(it, None) is None, "parameter count mismatch"
    return root


def _bincode(node):
    """bincode 1.3, fixed-width little-endian: struct = fields in order; Vec = u64 length +
    elements; usize = u64; f64 = IEEE bits; Option = u8 tag (+ value)."""
    kind, v = node
    if kind == "struct":
        return b"".join(_bincode(n) for _, n in v)
    if kind == "vecf":
        return struct.pack("<Q", len(v)) + struct.pack(f"<{len(v)}d", *v)
    if kind == "vecu":
        return struct.pack("<Q", len(v)) + struct.pack(f"<{len(v)}Q", *v)
    if kind == "u":
        return struct.pack("<Q", v)
    if kind == "f":
        return struct.pack("<d", v)
    if kind == "opt":
        return b"\x00" if v is None else b"\x01" + _bincode(v)
    raise AssertionError(kind)


def _jsonable(node):
    kind, v = node
    if kind == "struct":
        return {k: _jsonable(n) for k, n in v}
    if kind == "opt":
        return None if v is None else _jsonable(v)
    return v


def _ordered_keys(node):
    kind, v = node
    if kind == "struct":
        return [(k, _ordered_keys(n)) for k, n in v]
    if kind == "opt" and v is not None:
        return _ordered_keys(v)
    return None


def _pairs_keys(obj):
    if isinstance(obj, list) and obj and isinstance(obj[0], tuple):  # object_pairs_hook output
        return [(k, _pairs_keys(v)) for k, v in obj]
    return None


# ---------------------------------------------------------------------------
# Format pins
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("max_seq_len", [0, 256, 40])
def test_bincode_bytes_equal_the_independent_encoder(max_seq_len):
    c = cfg()
    p = params_for(c, 1)
    got = th.checkpoint_encode(c, p, th.CKPT_BINCODE, max_seq_len)
    want = _bincode(_tree(c, p, max_seq_len or 256))
    assert got == want


def test_bincode_known_bytes():
    # the first field of the file is backbone.embed.weight.data: u64 length 8 * 64 = 512, then
    # the first value's IEEE bits; the tail is critic_head.out_features = 1
    c = cfg()
    p = params_for(c, 2)
    b = th.checkpoint_encode(c, p)
    assert b[:8] == (512).to_bytes(8, "little")
    assert b[8:16] == struct.pack("<d", float(p[0]))
    assert b[-8:] == (1).to_bytes(8, "little")
    # embed.weight.shape follows its data: length 2, then 8 and 64
    o = 8 + 512 * 8
    assert b[o:o + 24] == struct.pack("<QQQ", 2, 8, 64)
    # embed.bias is Some: tag 1 and a 64-value tensor
    assert b[o + 24:o + 25] == b"\x01" and b[o + 25:o + 33] == (64).to_bytes(8, "little")


def test_json_document_matches_the_reference_tree():
    c = cfg()
    p = params_for(c, 3)
    text = th.checkpoint_encode(c, p, th.CKPT_JSON).decode()
    assert "\n" not in text and ": " not in text  # compact, as serde_json::to_writer
    doc = json.loads(text)
    tree = _tree(c, p)
    assert doc == _jsonable(tree)  # every value equal as f64, shapes and sizes equal
    pairs = json.loads(text, object_pairs_hook=lambda kv: kv)
    assert _pairs_keys(pairs) == _ordered_keys(tree)  # field names in declaration order
    assert doc["backbone"]["mla_layer"]["w_q"]["bias"] is None


def test_json_numbers_are_shortest_round_trip():
    c = cfg()
    p = params_for(c, 4)
    p[:6] = [0.1, -2.5e-8, 1e20, 3.0, -0.0, 123456.75]
    text = th.checkpoint_encode(c, p, th.CKPT_JSON).decode()
    data = text[text.index("[") + 1:text.index("]")].split(",")
    for s, v in zip(data, p):
        assert float(s) == float(v) and math.copysign(1, float(s)) == math.copysign(1, float(v))
        assert len(s.lstrip("-").replace(".", "").split("e")[0].strip("0")) <= len(repr(float(v)))
    assert data[0] == "0.10000000149011612"  # the f64 of fp32 0.1, shortest form
    assert data[3] == "3.0" and data[4] == "-0.0"


def test_rope_caches_follow_the_reference_formula():
    c = cfg()
    doc = json.loads(th.checkpoint_encode(c, params_for(c), th.CKPT_JSON, 8))
    rope = doc["backbone"]["mla_layer"]["rope"]
    assert rope["dim"] == 16 and rope["base"] == 10000.0
    assert len(rope["cos_cache"]) == 8 * 8
    for pos in range(8):
        for i in range(8):
            th_i = 1.0 / math.pow(10000.0, (2 * i) / 16)
            assert rope["cos_cache"][pos * 8 + i] == math.cos(pos * th_i)
            assert rope["sin_cache"][pos * 8 + i] == math.sin(pos * th_i)
    # RMSNorm eps is stored as the reference's f64 1e-5, not the widened fp32 1e-5f
    assert doc["backbone"]["norm_1"]["eps"] == 1e-5


# ---------------------------------------------------------------------------
# Round trips and reading files the library did not write
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("fmt", [th.CKPT_BINCODE, th.CKPT_JSON])
def test_round_trip_is_bit_exact(fmt):
    c = cfg()
    p = params_for(c, 5)
    p[7] = np.float32(np.nextafter(np.float32(1.0), np.float32(2.0)))
    p[8] = np.float32(1e-40)  # subnormal
    q = th.checkpoint_decode(c, th.checkpoint_encode(c, p, fmt), fmt)
    assert q.tobytes() == p.tobytes()


def test_decode_f64_values_round_to_nearest_fp32():
    c = cfg()
    p64 = workload.ppo_params(np.random.default_rng(6), c)  # float64, not fp32-representable
    b = _bincode(_tree(c, p64))
    assert np.array_equal(th.checkpoint_decode(c, b), p64.astype(np.float32))
    j = json.dumps(_jsonable(_tree(c, p64)), indent=1).encode()  # pretty-printed, Python's float repr
    assert np.array_equal(th.checkpoint_decode(c, j, th.CKPT_JSON), p64.astype(np.float32))


def test_json_reader_accepts_any_field_order_and_unknown_fields():
    c = cfg()
    p = params_for(c, 7)
    doc = _jsonable(_tree(c, p))
    bb = doc["backbone"]
    doc["backbone"] = dict(reversed(list(bb.items())))  # reversed field order
    doc["backbone"]["extra"] = {"anything": [1, 2, 3]}
    del doc["backbone"]["mla_layer"]["w_q"]["bias"]  # a missing Option is None
    q = th.checkpoint_decode(c, json.dumps(doc).encode(), th.CKPT_JSON)
    assert q.tobytes() == p.tobytes()


# ---------------------------------------------------------------------------
# Errors
# ---------------------------------------------------------------------------
def _code(fn, *a):
    with pytest.raises(th.TalosError) as e:
        fn(*a)
    return e.value.code


def test_configurations_the_format_cannot_hold():
    p = np.zeros(1, np.float32)
    for over in ({"attention": th.ATTN_MHA, "head_dim": 16}, {"n_layers": 2}, {"head_dim": 8}):
        c = cfg(**over)
        n = th.lib().talos_ppo_param_count(ctypes.byref(c))
        p = np.zeros(n, np.float32)
        assert _code(th.checkpoint_encode, c, p) == th.ERR_UNSUPPORTED, over
        assert _code(th.checkpoint_decode, c, b"") == th.ERR_UNSUPPORTED, over


def test_mismatched_checkpoints_are_rejected_and_params_untouched():
    c5 = cfg()
    b = th.checkpoint_encode(c5, params_for(c5, 8))
    c3 = cfg(n_actions=3)
    out = np.full(th.lib().talos_ppo_param_count(ctypes.byref(c3)), 7.0, np.float32)
    rc = th.lib().talos_ppo_checkpoint_decode(ctypes.byref(c3), b, len(b), th.CKPT_BINCODE, out.ctypes.data)
    assert rc == th.ERR_SHAPE and b"actor_head" in th.lib().talos_last_error()
    assert np.all(out == 7.0)
    c_eps = cfg(eps=1e-6)
    assert _code(th.checkpoint_decode, c_eps, b) == th.ERR_SHAPE
    c_base = cfg(rope_base=500.0)
    assert _code(th.checkpoint_decode, c_base, b) == th.ERR_SHAPE


def test_malformed_inputs():
    c = cfg()
    p = params_for(c, 9)
    b = th.checkpoint_encode(c, p)
    for cut in (0, 7, 100, len(b) - 1):
        assert _code(th.checkpoint_decode, c, b[:cut]) == th.ERR_FORMAT, cut
    o = 8 + 512 * 8 + 24  # embed.bias Option tag
    bad = b[:o] + b"\x02" + b[o + 1:]
    assert _code(th.checkpoint_decode, c, bad) == th.ERR_FORMAT
    # a huge Vec length must not be trusted
    assert _code(th.checkpoint_decode, c, (2 ** 62).to_bytes(8, "little") + b[8:]) in (th.ERR_SHAPE, th.ERR_FORMAT)
    doc = _jsonable(_tree(c, p))
    doc["backbone"]["embed"]["weight"]["data"][3] = None  # serde_json's NaN
    assert _code(th.checkpoint_decode, c, json.dumps(doc).encode(), th.CKPT_JSON) == th.ERR_FORMAT
    doc = _jsonable(_tree(c, p))
    del doc["backbone"]["norm_2"]
    assert _code(th.checkpoint_decode, c, json.dumps(doc).encode(), th.CKPT_JSON) == th.ERR_FORMAT
    doc = _jsonable(_tree(c, p))
    doc["backbone"]["mla_layer"]["rope"]["cos_cache"].pop()
    assert _code(th.checkpoint_decode, c, json.dumps(doc).encode(), th.CKPT_JSON) == th.ERR_FORMAT
    doc = _jsonable(_tree(c, p))
    doc["backbone"]["embed"]["in_features"] = 8.0  # a usize must be an integer
    assert _code(th.checkpoint_decode, c, json.dumps(doc).encode(), th.CKPT_JSON) == th.ERR_FORMAT
    for text in (b"{", b"[1,2", b'{"backbone":}', b"{} x", b'{"a":tru}'):
        assert _code(th.checkpoint_decode, c, text, th.CKPT_JSON) == th.ERR_FORMAT, text


def test_non_finite_values_follow_the_reference_writers():
    c = cfg()
    p = params_for(c, 10)
    p[0] = np.nan
    # bincode keeps them, serde_json writes null (and its reader rejects the file)
    q = th.checkpoint_decode(c, th.checkpoint_encode(c, p))
    assert np.isnan(q[0]) and np.array_equal(q[1:], p[1:])
    text = th.checkpoint_encode(c, p, th.CKPT_JSON)
    assert text.startswith(b'{"backbone":{"embed":{"weight":{"data":[null,')
    assert _code(th.checkpoint_decode, c, text, th.CKPT_JSON) == th.ERR_FORMAT


# ---------------------------------------------------------------------------
# Files: save_ppo_model / load_ppo_model
# ---------------------------------------------------------------------------
def test_save_writes_both_files_and_load_prefers_the_binary(tmp_path):
    c = cfg()
    p = params_for(c, 11)
    path = str(tmp_path / "ppo.cache")
    th.save_ppo_model(c, p, path)
    assert os.path.exists(path + ".bin") and os.path.exists(path)
    assert not any(f.endswith(".tmp") for f in os.listdir(tmp_path))
    assert open(path + ".bin", "rb").read() == th.checkpoint_encode(c, p)
    assert open(path, "rb").read() == th.checkpoint_encode(c, p, th.CKPT_JSON)
    assert th.load_ppo_model(c, path).tobytes() == p.tobytes()
    # a different model in the JSON file: the binary wins
    p2 = params_for(c, 12)
    open(path, "wb").write(th.checkpoint_encode(c, p2, th.CKPT_JSON))
    assert th.load_ppo_model(c, path).tobytes() == p.tobytes()


def test_load_falls_back_to_json(tmp_path):
    c = cfg()
    p = params_for(c, 13)
    path = str(tmp_path / "m")
    open(path, "wb").write(th.checkpoint_encode(c, p, th.CKPT_JSON))
    assert th.load_ppo_model(c, path).tobytes() == p.tobytes()  # no binary
    open(path + ".bin", "wb").write(b"\x01\x02")  # a binary that does not decode
    assert th.load_ppo_model(c, path).tobytes() == p.tobytes()
    os.remove(path)
    assert _code(th.load_ppo_model, c, path) == th.ERR_FORMAT  # only the bad binary is left
    os.remove(path + ".bin")
    assert _code(th.load_ppo_model, c, path) == th.ERR_IO
    assert _code(th.save_ppo_model, c, p, str(tmp_path / "no" / "such" / "dir")) == th.ERR_IO
