"""Host-only formats against the reference compiled from its sources
(oracle/_ref/libref.so): the .conf parser (tensor.c:145-266) and NCMT
training rows (tensor.c:375-395).  Both libraries fill the same struct
layout, so their outputs are compared byte for byte."""
import ctypes
import os
import struct

import numpy as np
import pytest

import ncmhip
import oracle as O

pytestmark = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref/libref.so not built")


@pytest.fixture(scope="module")
def libs():
    ours = ncmhip.bind(ncmhip.load(), ncmhip.FORMAT_SIGS)
    ref = ncmhip.bind(O.ref(), ncmhip.FORMAT_SIGS)
    return ours, ref


def load_conf(lib, path):
    buf = ctypes.create_string_buffer(4096)  # larger than NCMConfig: a size mismatch shows in the tail
    rc = lib.config_load(buf, path.encode())
    return rc, buf.raw


CONFS = {
    "ncp": "task=sudoku\nmodel.n_layer=4\nmodel.n_head=4\nmodel.n_embd=256\nmodel.context_length=81\n"
           "model.vocab_size=16,16, 32 ,64\nmodel.use_rope=True\nmodel.rope_base=10000\nmodel.use_swiglu=1\n"
           "model.bias=0\nmodel.n_kv_heads=2\nmodel.attn_pattern=block_diagonal\nmodel.dropout=0.1\n",
    "qwen": "task=lm\nmodel.n_layer=24\nmodel.n_head=14\nmodel.n_embd=896\nmodel.context_length=8192\n"
            "model.rope_theta=1000000.0\nmodel.n_kv_heads=2\nmodel.vocab_size=151936\ntok.kind=hf\n"
            "tok.model_id=Qwen/Qwen2.5-0.5B\ntok.eos_id=151643\ntok.pad_id=False\ngen.temperature=0.7\n"
            "gen.top_k=40\ngen.top_p=0.95\n",
    "vq": "vq.embed_dim=256\nvq.levels=1,2,4, 8,16\nvq.vocab=4096,4096,4096\nvq.soft_tau=0.25\nvq.qr_ratio=0.5\n"
          "vq.qr_enabled=1\nvq.l1_norm=t\nvq.l1_norm_final= F\nvq.qk_norm=2\nvq.enc_window=64\nvq.pre_quant_gn=1\n"
          "model.attn_pattern=block_causal\nmodel.tie_heads_learn_scale=T\nmodel.layerscale_init=1e-4\n",
    "edge": "no equals sign here\n=empty key\nunknown.key=5\nmodel.n_head=  7\nmodel.n_layer=x12\n"
            "model.n_embd=12abc\r\ntask=" + "t" * 100 + "\ngen.adj=0.5,3,0.25\nmodel.prefix_pad_token_id=-3\n"
            "tok.model_id=" + "m" * 1100 + "\nmodel.vocab_size=" + ",".join(str(i) for i in range(80)) + "\n",
    "adj1": "gen.adj=1.5\n",
    "adj2": "gen.adj=2,7\n",
    "adjempty": "gen.adj=\nmodel.n_head=3\n",
    "defaults": "",
}


@pytest.mark.parametrize("name", sorted(CONFS))
def test_config_load_matches_reference(libs, tmp_path, name):
    path = tmp_path / f"{name}.conf"
    path.write_bytes(CONFS[name].encode())
    (rc1, b1), (rc2, b2) = load_conf(libs[0], str(path)), load_conf(libs[1], str(path))
    assert rc1 == rc2 == 0
    assert b1 == b2
    c = ncmhip.NCMConfig.from_buffer_copy(b1[:ctypes.sizeof(ncmhip.NCMConfig)])
    if name == "ncp":
        assert (c.n_layer, c.n_embd, c.n_kv_heads, c.bias, c.n_levels_out) == (4, 256, 2, 0, 4)
        assert list(c.vocab_size[:4]) == [16, 16, 32, 64] and c.use_rope == 1
    if name == "defaults":  # python-style defaults, n_kv_heads falls back to n_head
        assert (c.bias, c.rope_base, c.rope_theta, c.n_kv_heads, c.gen_top_k) == (1, 10000, 10000.0, 0, 1)
        assert (c.eos_token_id, c.pad_token_id, c.attn_pattern_block_diag) == (-1, -1, 1)
    if name == "edge":
        assert c.n_head == 7 and c.n_levels_out == 64 and len(c.task) == 63
        assert (c.gen_adj_a, c.gen_adj_w, c.gen_adj_d) == (0.5, 3, 0.25)


def test_config_missing_file(libs, tmp_path):
    p = str(tmp_path / "absent.conf")
    assert load_conf(libs[0], p)[0] == load_conf(libs[1], p)[0] == -1


def write_ncmt(path, rows, magic=b"NCMT", short=0):
    rows = np.asarray(rows, np.int32)
    data = rows.tobytes()
    path.write_bytes(magic + struct.pack("<QQ", rows.shape[0], rows.shape[1]) + data[:len(data) - short])


def read_rows(lib, path, max_rows):
    p = lib.train_data_load(str(path).encode(), max_rows)
    if not p:
        return None
    d = ncmhip.TrainData.from_address(p)
    n = d.n_rows * d.row_len
    out = (d.n_rows, d.row_len, np.ctypeslib.as_array(d.rows, (n,)).copy() if n else np.zeros(0, np.int32))
    lib.train_data_free(p)
    return out


@pytest.mark.parametrize("case", ["full", "capped", "cap_above", "empty", "bad_magic", "short"])
def test_train_data_matches_reference(libs, tmp_path, case):
    rng = np.random.default_rng(3)
    rows = rng.integers(-5, 50000, (37, 19))
    path = tmp_path / "d.nctrain"
    max_rows = {"capped": 10, "cap_above": 100}.get(case, 0)
    if case == "empty":
        rows = np.zeros((0, 19), np.int32)
    write_ncmt(path, rows, magic=b"NCMX" if case == "bad_magic" else b"NCMT", short=4 if case == "short" else 0)
    a, b = read_rows(libs[0], path, max_rows), read_rows(libs[1], path, max_rows)
    if case in ("bad_magic", "short"):
        assert a is None and b is None
        return
    assert a[:2] == b[:2] and np.array_equal(a[2], b[2])
    want = rows[:max_rows] if case == "capped" else rows
    assert a[:2] == want.shape and np.array_equal(a[2], want.ravel())
