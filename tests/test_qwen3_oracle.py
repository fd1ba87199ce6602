"""Qwen3 text encoder oracle (oracle/orc_qwen3.c) against the reference's own
qwen3_forward (iris_qwen3.c, compiled from its sources into oracle/_ref) on a
random-init model written in the HuggingFace layout, and against properties
fixed by the mathematics (causality, padding). CPU only."""
import ctypes
import os

import numpy as np
import pytest

import iris_testlib as tl

LAYERS = 28          # the Flux extraction reads layer 26


@pytest.fixture(scope="module")
def qdir(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("qwen3_tiny"))
    tl.write_qwen3_dir(d, layers=LAYERS, seed=3)
    return d


@pytest.fixture(scope="module")
def orc():
    return tl.oracle()


@pytest.fixture(scope="module")
def oq(orc, qdir):
    m = ctypes.c_void_p(orc.orc_qwen3_load(qdir.encode()))
    assert m.value
    yield m
    orc.orc_qwen3_free(m)


def ids_mask(seq, n_real, seed, vocab=300):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, vocab, seq).astype(np.int32)
    ids[n_real:] = 151643 % vocab            # any id; the mask hides these keys
    mask = np.zeros(seq, np.int32)
    mask[:n_real] = 1
    return ids, mask


def run_oracle(orc, m, ids, mask, mode, last=-1):
    orc.orc_qwen3_set_mode(m, mode)
    dims = (ctypes.c_int * 4)()
    orc.orc_qwen3_dims(m, dims)
    seq = len(ids)
    width = dims[0] if last >= 0 else dims[2]
    p = orc.orc_qwen3_forward(m, ids.ctypes.data_as(tl.IP), None if mask is None else mask.ctypes.data_as(tl.IP),
                              seq, last)
    assert p
    return tl.take_f32(orc, p, seq * width).reshape(seq, width)


@pytest.mark.skipif(not os.path.exists(tl.REF_SO), reason="reference build (oracle/_ref) not present")
@pytest.mark.parametrize("mode,seq,n_real", [(0, 24, 19), (1, 24, 24), (0, 70, 70)])
def test_oracle_vs_reference(orc, oq, qdir, mode, seq, n_real):
    ref = tl.ref()
    rm = ctypes.c_void_p(ref.qwen3_model_load(qdir.encode()))
    assert rm.value
    enc = tl.Qwen3Encoder(None, rm.value)
    ref.qwen3_set_extraction_mode(ctypes.byref(enc), mode)
    ids, mask = ids_mask(seq, n_real, 10 + seq)
    width = 256 * (1 if mode else 3)
    p = ref.qwen3_forward(rm, ids.ctypes.data_as(tl.IP), mask.ctypes.data_as(tl.IP), seq)
    assert p
    want = tl.take_f32(ref, p, seq * width).reshape(seq, width)
    ref.qwen3_model_free(rm)
    got = run_oracle(orc, oq, ids, mask, mode)
    assert np.all(np.isfinite(want)) and want.std() > 0.1
    assert tl.rel_l2(got, want) < 1e-4


def test_causality_and_padding(orc, oq):
    """Row r depends only on tokens 0..r: a prefix of the sequence gives the
    same rows; tokens behind the padding mask change nothing."""
    ids, _ = ids_mask(40, 40, 5)
    full = run_oracle(orc, oq, ids, None, 1)
    head = run_oracle(orc, oq, ids[:25].copy(), None, 1)
    assert tl.rel_l2(head, full[:25]) < 1e-6
    ids2 = ids.copy()
    ids2[30:] = (ids2[30:] + 7) % 300
    mask = np.r_[np.ones(30, np.int32), np.zeros(10, np.int32)]
    a = run_oracle(orc, oq, ids, mask, 1)
    b = run_oracle(orc, oq, ids2, mask, 1)
    assert np.array_equal(a[:30], b[:30])
    assert tl.rel_l2(a[:30], full[:30]) < 1e-6


def read_safetensors(path):
    import json
    import struct
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        hdr = json.loads(f.read(n))
        data = f.read()
    out = {}
    for k, v in hdr.items():
        if k == "__metadata__":
            continue
        a, b = v["data_offsets"]
        assert v["dtype"] == "BF16"
        out[k] = tl.bf16_to_f32(np.frombuffer(data[a:b], np.uint16)).astype(np.float64).reshape(v["shape"])
    return out


def np_layer(W, i, h, heads, kv_heads, mask=None):
    """One Qwen3 decoder layer in float64 from the textbook definitions."""
    p = f"model.layers.{i}."
    seq, hd = h.shape[0], 128

    def rms(x, w):
        return x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6) * w

    x = rms(h, W[p + "input_layernorm.weight"])
    q = (x @ W[p + "self_attn.q_proj.weight"].T).reshape(seq, heads, hd)
    k = (x @ W[p + "self_attn.k_proj.weight"].T).reshape(seq, kv_heads, hd)
    v = (x @ W[p + "self_attn.v_proj.weight"].T).reshape(seq, kv_heads, hd)
    q, k = rms(q, W[p + "self_attn.q_norm.weight"]), rms(k, W[p + "self_attn.k_norm.weight"])
    ang = np.arange(seq)[:, None] * (1e6 ** (-np.arange(64) * 2.0 / hd))[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]

    def rot(t):
        a, b = t[..., :64], t[..., 64:]
        return np.concatenate([a * c - b * s, a * s + b * c], -1)

    q, k = rot(q), rot(k)
    out = np.zeros((seq, heads, hd))
    allowed = np.tril(np.ones((seq, seq), bool))
    if mask is not None:
        allowed &= mask[None, :].astype(bool)
    for hh in range(heads):
        kv = hh // (heads // kv_heads)
        sc = q[:, hh] @ k[:, kv].T / np.sqrt(hd)
        sc = np.where(allowed, sc, -np.inf)
        pr = np.exp(sc - sc.max(1, keepdims=True))
        pr /= pr.sum(1, keepdims=True)
        out[:, hh] = pr @ v[:, kv]
    h = h + out.reshape(seq, heads * hd) @ W[p + "self_attn.o_proj.weight"].T
    x = rms(h, W[p + "post_attention_layernorm.weight"])
    g, u = x @ W[p + "mlp.gate_proj.weight"].T, x @ W[p + "mlp.up_proj.weight"].T
    return h + (g / (1 + np.exp(-g)) * u) @ W[p + "mlp.down_proj.weight"].T


def test_two_layers_known_answer(orc, oq, qdir):
    """Layers 0 and 1 of the oracle against a float64 numpy restatement of the
    decoder layer with the weights read back from the same file, with a
    padding mask: pins the oracle independently of the reference."""
    W = read_safetensors(os.path.join(qdir, "model-00001-of-00001.safetensors"))
    seq = 20
    ids, mask = ids_mask(seq, 15, 8)
    h = W["model.embed_tokens.weight"][ids]
    for i in range(2):
        h = np_layer(W, i, h, 4, 2, mask)
    got = run_oracle(orc, oq, ids, mask, 1, last=1)
    assert tl.rel_l2(got, h) < 1e-5
