"""The weight container reader (apus_hip_st_*, the counterpart of the
reference's c/st.h:64-89) and the layer loaders.

Containers are written in-test by an independent writer (the installed
`safetensors` package): one shard, and a directory with
model.safetensors.index.json over two shards, under the reference's
tensor names (c/model.h:440-490). CPU: every tensor's dtype, shape and
payload bytes read back exactly; broken files (truncated payload, header
length past the end, a name the index puts in the wrong shard, a missing
tensor) are refused with an error. GPU: the layer loaders put one GDN and
one GQA layer's hot weights on the device, and a decode step with the
loaded layers equals, bit for bit, the same step with the weights uploaded
directly.
"""
import json
import os

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import apus_hip
import synth

GD = synth.GDN_DIMS
AD = synth.ATTN_DIMS
P = "model.language_model.layers.{}."


def _tensors(rng, a_log_bf16=False):
    """GDN layer 0 and full-attention layer 3 (plus an unrelated tensor)."""
    hk, hv, dk, dv = GD
    cd = 2 * hk * dk + hv * dv
    w = synth.gdn_weights(rng)
    aw = synth.attn_weights(rng)
    bf = lambda codes: torch.from_numpy(codes.view(np.int16)).view(torch.bfloat16)
    t = {P.format(0) + "linear_attn.conv1d.weight": bf(w["conv_w"]).reshape(cd, 1, 4),
         P.format(0) + "linear_attn.norm.weight": bf(w["onorm_w"]),
         P.format(0) + "linear_attn.A_log": torch.from_numpy(w["A_log"]),
         P.format(0) + "linear_attn.dt_bias": torch.from_numpy(w["dt_bias"]),
         P.format(3) + "self_attn.q_norm.weight": bf(aw["qn_w"]),
         P.format(3) + "self_attn.k_norm.weight": bf(aw["kn_w"]),
         "model.language_model.norm.weight": torch.ones(16, dtype=torch.float32),
         "extra.i64": torch.arange(5, dtype=torch.int64)}
    if a_log_bf16:
        # a BF16 container (the real checkpoint is pure BF16): A_log widened
        t[P.format(0) + "linear_attn.A_log"] = t[P.format(0) + "linear_attn.A_log"].to(torch.bfloat16)
        w["A_log"] = t[P.format(0) + "linear_attn.A_log"].to(torch.float32).numpy()
    return t, w, aw


def _raw(t):
    return t.contiguous().view(torch.uint8).numpy().reshape(-1) if t.dtype != torch.bfloat16 else \
        t.contiguous().view(torch.int16).numpy().view(np.uint8).reshape(-1)


def _write_dir(tmp_path, t):
    names = sorted(t)
    a, b = names[::2], names[1::2]
    save_file({n: t[n] for n in a}, str(tmp_path / "model-00001-of-00002.safetensors"))
    save_file({n: t[n] for n in b}, str(tmp_path / "model-00002-of-00002.safetensors"))
    wm = {n: "model-00001-of-00002.safetensors" for n in a}
    wm.update({n: "model-00002-of-00002.safetensors" for n in b})
    (tmp_path / "model.safetensors.index.json").write_text(
        json.dumps({"metadata": {"total_size": 0}, "weight_map": wm}))


def _check_all(c, t):
    assert len(c) == len(t)
    for n, x in t.items():
        info = c.find(n)
        assert info["shape"] == tuple(x.shape), n
        assert info["dtype"] == {torch.bfloat16: "BF16", torch.float32: "F32",
                                 torch.int64: "I64"}[x.dtype], n
        assert np.array_equal(c.read(n), _raw(x)), n


def test_single_shard_roundtrip(tmp_path):
    t, _, _ = _tensors(np.random.default_rng(41))
    save_file(t, str(tmp_path / "one.safetensors"), metadata={"format": "pt"})
    c = apus_hip.Container(tmp_path / "one.safetensors")
    _check_all(c, t)
    with pytest.raises(apus_hip.ApusHipError):
        c.find("no.such.tensor")
    c.close()


def test_index_directory_roundtrip(tmp_path):
    t, _, _ = _tensors(np.random.default_rng(42))
    _write_dir(tmp_path, t)
    c = apus_hip.Container(tmp_path)
    _check_all(c, t)
    c.close()


def test_broken_containers_refused(tmp_path):
    t, _, _ = _tensors(np.random.default_rng(43))
    f = tmp_path / "one.safetensors"
    save_file(t, str(f))
    data = f.read_bytes()
    (tmp_path / "trunc.safetensors").write_bytes(data[:-100])          # payload cut short
    (tmp_path / "hdr.safetensors").write_bytes((len(data)).to_bytes(8, "little") + data[8:])
    (tmp_path / "json.safetensors").write_bytes(data[:9] + b"{" + data[10:])    # bad JSON
    for bad in ("trunc", "hdr", "json"):
        with pytest.raises(apus_hip.ApusHipError):
            apus_hip.Container(tmp_path / f"{bad}.safetensors")
    d = tmp_path / "d"
    d.mkdir()
    _write_dir(d, t)
    idx = json.loads((d / "model.safetensors.index.json").read_text())
    first = sorted(t)[0]
    idx["weight_map"][first] = "model-00002-of-00002.safetensors"        # wrong shard
    (d / "model.safetensors.index.json").write_text(json.dumps(idx))
    with pytest.raises(apus_hip.ApusHipError):
        apus_hip.Container(d)


def _hand_written(path, entry, payload=b"\0" * 64):
    """A container whose header is written by hand (one tensor "x")."""
    hdr = json.dumps({"x": entry}).encode()
    path.write_bytes(len(hdr).to_bytes(8, "little") + hdr + payload)


@pytest.mark.parametrize("entry", [
    # element count overflows 64 bits (2^40 x 2^40 x 2^40), a payload of 8 bytes
    {"dtype": "BF16", "shape": [2 ** 40, 2 ** 40, 2 ** 40], "data_offsets": [0, 8]},
    # 2^63 x 2 wraps to 0 bytes with an unchecked multiply
    {"dtype": "BF16", "shape": [2 ** 53 - 1, 2 ** 10], "data_offsets": [0, 0]},
    # non-integral dimension and offsets
    {"dtype": "BF16", "shape": [2.5], "data_offsets": [0, 5]},
    {"dtype": "U8", "shape": [4], "data_offsets": [0.5, 4.5]},
    # offsets past 2^53 (not exact as JSON doubles) and past the file
    {"dtype": "U8", "shape": [8], "data_offsets": [2 ** 60, 2 ** 60 + 8]},
    {"dtype": "U8", "shape": [8], "data_offsets": [60, 68]},
    # negative dimension
    {"dtype": "U8", "shape": [-8], "data_offsets": [0, 8]},
])
def test_header_numbers_refused(tmp_path, entry):
    """Dimensions and offsets must be integers below 2^53 and the element
    count and byte size must not overflow: a crafted header is refused
    rather than reporting a bogus shape or reading past the payload."""
    f = tmp_path / "x.safetensors"
    _hand_written(f, entry)
    with pytest.raises(apus_hip.ApusHipError):
        apus_hip.Container(f)


def test_hand_written_header_accepted(tmp_path):
    f = tmp_path / "x.safetensors"
    _hand_written(f, {"dtype": "U8", "shape": [2, 4], "data_offsets": [8, 16]})
    c = apus_hip.Container(f)
    assert c is not None


@pytest.mark.gpu
@pytest.mark.parametrize("a_log_bf16", [False, True])
def test_layer_loaders(tmp_path, hip, a_log_bf16):
    rng = np.random.default_rng(44)
    t, w, aw = _tensors(rng, a_log_bf16)
    _write_dir(tmp_path, t)
    c = apus_hip.Container(tmp_path)
    Lg = c.gdn_layer(0, GD)
    La = c.attn_layer(3, AD)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16) if a.dtype == np.uint16
                                     else np.ascontiguousarray(a)).cuda()
    Lg2 = hip.gdn_layer(GD, {n: dev(a) for n, a in w.items()})
    La2 = hip.attn_layer(AD, {n: dev(a) for n, a in aw.items()})
    # one GDN decode token over 2 sequences, with each layer struct
    hk, hv, dk, dv = GD
    tok = synth.gdn_tokens(rng, 2)
    conv, S = synth.gdn_state(rng, 2)
    tt = {n: dev(a) for n, a in tok.items()}
    ys = []
    for L in (Lg, Lg2):
        dconv, dS = dev(conv), torch.empty(S.shape, dtype=torch.float32, device="cuda")
        hip.gdn_state_pack(dev(S), dS)
        y = torch.empty((2, hv * dv), dtype=torch.int16, device="cuda")
        hip.gdn_decode(L, [0, 1, 2], tt["qkv"], tt["z"], tt["a"], tt["b"], dconv, dS, y)
        ys.append((y, dconv, dS))
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(ys[0], ys[1]))
    # one attention verify step
    nh, nkv, d, rot, theta = AD
    atok = synth.attn_tokens(rng, 3)
    at = {n: dev(a) for n, a in atok.items()}
    outs = []
    for L in (La, La2):
        kc = torch.zeros((2, nkv, 64, d), dtype=torch.int16, device="cuda")
        vc = torch.zeros_like(kc)
        y = torch.empty((3, nh * d), dtype=torch.int16, device="cuda")
        hip.attn_decode(L, [0, 2, 3], [10, 4], at["qg"], at["k"], at["v"], kc, vc, 64, y)
        outs.append((y, kc, vc))
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(outs[0], outs[1]))
    apus_hip.free_gdn_layer(Lg)
    apus_hip.free_attn_layer(La)
    c.close()
