"""NCM1 weight files, the AdamW object and NCK1 checkpoints on the device,
against the reference compiled from its sources (oracle/_ref/libref.so, whose
tensors are host memory): files written by either side load in the other,
AdamW steps are bit-identical, and a checkpoint of the same state is the same
file byte for byte.  The refusal cases follow the reference's own
tests/ckpt_unit.c and test_ckpt.sh (truncation, bit flips, identity
mismatches); both libraries must refuse each one, and this library must leave
the live weights, moments and step untouched."""
import ctypes
import os
import struct

import numpy as np
import pytest

import ncmhip
import oracle as O

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref/libref.so not built")]

MEM = {k: ncmhip._SIGS[k] for k in ("tensor_alloc", "tensor_free", "mem_h2d", "mem_d2h")}
ERR = 512


@pytest.fixture(scope="module")
def libs():
    ncmhip.init(0)
    print("[gpu] format tests on device 0", flush=True)
    ours = ncmhip.bind(ncmhip.load(), ncmhip.FORMAT_SIGS)
    ref = ncmhip.bind(O.ref(), {**ncmhip.FORMAT_SIGS, **MEM})
    return ours, ref


def tensors_spec(seed=0):
    rng = np.random.default_rng(seed)
    return [("wte.weight", rng.standard_normal((17, 8)).astype(np.float32)),
            ("blk.0.attn.bias", rng.standard_normal(8).astype(np.float32)),
            ("blk.0.conv.weight", rng.standard_normal((2, 3, 4, 5)).astype(np.float32)),
            ("scale", np.array(1.5, np.float32).reshape(())),
            ("blk.0.mlp.weight", rng.standard_normal((16, 8)).astype(np.float32))]


class Store:
    """A WeightStore built from Python (items owned here; tensors via lib)."""

    def __init__(self, lib, spec):
        self.lib = lib
        self.items = (ncmhip.NamedTensor * len(spec))()
        for i, (name, arr) in enumerate(spec):
            shape = (ncmhip.i64 * 4)(*arr.shape, *([0] * (4 - arr.ndim)))
            t = lib.tensor_alloc(arr.ndim, shape)
            assert t
            self.items[i].name = name.encode()
            self.items[i].t = ctypes.cast(t, ctypes.POINTER(ncmhip.TensorS))
            a = np.ascontiguousarray(arr, np.float32)
            lib.mem_h2d(self.items[i].t.contents.data, a.ctypes.data, a.nbytes)
        self.ws = ncmhip.WeightStore(self.items, len(spec))

    def ptr(self):
        return ctypes.addressof(self.ws)

    def free(self):
        for i in range(self.ws.count):
            self.lib.tensor_free(ctypes.cast(self.items[i].t, ctypes.c_void_p))


def read_store(lib, ws):
    out = []
    for i in range(ws.count):
        t = ws.items[i].t.contents
        a = np.empty(t.n, np.float32)
        lib.mem_d2h(a.ctypes.data, t.data, a.nbytes)
        out.append((ws.items[i].name.decode(), a.reshape(tuple(t.shape[:t.ndim]))))
    return out


def same(a, b):
    return len(a) == len(b) and all(n1 == n2 and x.shape == y.shape and np.array_equal(x.view(np.uint32), y.view(np.uint32))
                                    for (n1, x), (n2, y) in zip(a, b))


def dev_read(lib, p, n):
    a = np.empty(n, np.float32)
    lib.mem_d2h(a.ctypes.data, p, a.nbytes)
    return a


def test_ncm1_round_trips_with_reference(libs, tmp_path):
    ours, ref = libs
    spec = tensors_spec(1)
    for writer, reader in ((ours, ref), (ref, ours), (ours, ours)):
        s = Store(writer, spec)
        path = str(tmp_path / "w.ncm").encode()
        assert writer.weights_save(s.ptr(), path) == 0
        ws = ncmhip.WeightStore()
        assert reader.weights_load(ctypes.byref(ws), path) == 0
        assert same(read_store(reader, ws), [(n, a) for n, a in spec])
        assert ws.names() == [n for n, _ in spec]
        t = reader.weights_get(ctypes.byref(ws), b"blk.0.attn.bias")
        assert t and ctypes.cast(t, ctypes.POINTER(ncmhip.TensorS)).contents.n == 8
        assert not reader.weights_get(ctypes.byref(ws), b"missing")
        reader.weights_free(ctypes.byref(ws))
        s.free()
    # identical bytes from both writers
    s1, s2 = Store(ours, spec), Store(ref, spec)
    assert ours.weights_save(s1.ptr(), str(tmp_path / "a.ncm").encode()) == 0
    assert ref.weights_save(s2.ptr(), str(tmp_path / "b.ncm").encode()) == 0
    assert (tmp_path / "a.ncm").read_bytes() == (tmp_path / "b.ncm").read_bytes()
    s1.free(), s2.free()


def test_ncm1_rejects_bad_files(libs, tmp_path):
    ours, ref = libs
    s = Store(ours, tensors_spec(2))
    good = tmp_path / "g.ncm"
    assert ours.weights_save(s.ptr(), str(good).encode()) == 0
    s.free()
    raw = good.read_bytes()
    # byte 29 is the second byte of the first tensor's u64 byte count (544 -> 800)
    cases = {"magic": b"XCM1" + raw[4:], "truncated": raw[:-3], "size": raw[:29] + b"\x03" + raw[30:]}
    for name, data in cases.items():
        p = tmp_path / f"{name}.ncm"
        p.write_bytes(data)
        ws = ncmhip.WeightStore()
        assert ours.weights_load(ctypes.byref(ws), str(p).encode()) == -1, name
        assert ws.count == 0 and not ws.items  # nothing left allocated
    ws = ncmhip.WeightStore()
    assert ours.weights_load(ctypes.byref(ws), str(tmp_path / "absent.ncm").encode()) == -1


def make_opt(lib, store, lr_mult):
    o = ctypes.cast(lib.adamw_new(store.ptr(), None), ctypes.POINTER(ncmhip.AdamW))
    assert o
    o.contents.wd = 0.1
    for i, m in enumerate(lr_mult):
        o.contents.lr[i] = m
    return o


def run_steps(lib, o, grads, steps):
    for s in range(steps):
        for i, g in enumerate(grads[s]):
            lib.mem_h2d(o.contents.g[i], g.ctypes.data, g.nbytes)
        lib.adamw_step(o, 3e-4, 2.0, 10.0)


def opt_state(lib, o):
    c = o.contents
    return [(dev_read(lib, c.params[i], c.sizes[i]), dev_read(lib, c.m[i], c.sizes[i]),
             dev_read(lib, c.v[i], c.sizes[i])) for i in range(c.n)], c.step


def both_trained(libs, spec, lr_mult, steps=3, seed=5):
    rng = np.random.default_rng(seed)
    grads = [[rng.standard_normal(a.size).astype(np.float32) for _, a in spec] for _ in range(steps)]
    out = []
    for lib in libs:
        s = Store(lib, spec)
        o = make_opt(lib, s, lr_mult)
        run_steps(lib, o, grads, steps)
        out.append((s, o))
    return out


def test_adamw_object_matches_reference(libs):
    """adamw_new / adamw_step over a store: params, moments and step counter
    bit-identical to the reference's host loop (train.c:102-145)."""
    spec = tensors_spec(3)
    (s1, o1), (s2, o2) = both_trained(libs, spec, [1.0, 0.5, 2.0, 1.0, 0.25])
    st1, k1 = opt_state(libs[0], o1)
    st2, k2 = opt_state(libs[1], o2)
    assert k1 == k2 == 3
    for a, b in zip(st1, st2):
        for x, y in zip(a, b):
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    libs[0].adamw_zero_grad(o1)
    ncmhip.sync()
    assert not dev_read(libs[0], o1.contents.g[0], o1.contents.sizes[0]).any()
    libs[0].adamw_free(o1), libs[1].adamw_free(o2)
    s1.free(), s2.free()


def run_state(**kw):
    rs = ncmhip.CkptRunState(global_step=7, batch_rng=0x9E3779B97F4A7C15, base_lr=3e-4, warmup=2.0, total=10.0,
                             batch_B=32, accum_pending=0, n_rows=5000, row_len=513, data_hash=0x1234567890ABCDEF,
                             data_path=b"data/train.nctrain", conf_hash=0xFEDCBA0987654321, tokenizer_id=b"gpt2",
                             noise_sd=0.0, train_cfg_json=b'{"lr":3e-4,"B":32}')
    for k, v in kw.items():
        setattr(rs, k, v)
    return rs


def expect(**kw):
    ex = ncmhip.CkptExpect(batch_B=32, n_rows=5000, row_len=513, data_hash=0x1234567890ABCDEF,
                           conf_hash=0xFEDCBA0987654321, tokenizer_id=b"gpt2", base_lr=3e-4, warmup=2.0, total=10.0,
                           b1=0.9, b2=0.95, eps=1e-8, wd=0.1)
    for k, v in kw.items():
        setattr(ex, k, v)
    return ex


def save(lib, s, o, rs, path):
    err = ctypes.create_string_buffer(ERR)
    rc = lib.ckpt_save_atomic(s.ptr(), o, ctypes.byref(rs), str(path).encode(), err, ERR)
    return rc, err.value.decode()


def load(lib, s, o, ex, path):
    err = ctypes.create_string_buffer(ERR)
    out = ncmhip.CkptRunState()
    rc = lib.ckpt_load_training(str(path).encode(), s.ptr(), o, ctypes.byref(ex), ctypes.byref(out), err, ERR)
    return rc, err.value.decode(), out


def fnv1a(data):
    h = 14695981039346656037
    for b in data:
        h = ((h ^ b) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h


def test_nck1_is_the_reference_file(libs, tmp_path):
    ours, ref = libs
    spec = tensors_spec(4)
    lr_mult = [1.0, 0.5, 2.0, 1.0, 0.25]
    (s1, o1), (s2, o2) = both_trained(libs, spec, lr_mult)
    rs = run_state()
    a, b = tmp_path / "ours.nckpt", tmp_path / "ref.nckpt"
    assert save(ours, s1, o1, rs, a) == (0, "")
    assert save(ref, s2, o2, rs, b)[0] == 0
    assert a.read_bytes() == b.read_bytes()
    assert not [p for p in os.listdir(tmp_path) if ".tmp." in p]
    raw = a.read_bytes()
    assert struct.unpack("<Q", raw[-8:])[0] == fnv1a(raw[:-8])
    n1, n2 = ctypes.c_uint64(), ctypes.c_uint64()
    assert ours.ckpt_file_hash(str(a).encode(), ctypes.byref(n1)) == ref.ckpt_file_hash(str(a).encode(), ctypes.byref(n2))
    assert n1.value == n2.value == len(raw)
    for p, want in ((a, 1), (tmp_path / "absent", -1)):
        assert ours.ckpt_probe(str(p).encode()) == ref.ckpt_probe(str(p).encode()) == want
    # cross loads: fresh stores of the same names/shapes, fresh optimizers
    zero = [(n, np.zeros_like(x)) for n, x in spec]
    want_state, want_step = opt_state(ours, o1)
    trained = read_store(ours, s1.ws)  # the checkpoint holds the weights after the steps
    for lib, path in ((ours, b), (ref, a)):
        s = Store(lib, zero)
        o = make_opt(lib, s, lr_mult)
        rc, err, out = load(lib, s, o, expect(), path)
        assert rc == 0, err
        assert same(read_store(lib, s.ws), trained)
        got, step = opt_state(lib, o)
        assert step == want_step == 3
        for x, y in zip(got, want_state):
            for u, w in zip(x[1:], y[1:]):
                assert np.array_equal(u.view(np.uint32), w.view(np.uint32))
        assert (out.global_step, out.batch_rng, out.n_rows, out.row_len) == (7, 0x9E3779B97F4A7C15, 5000, 513)
        assert not out.data_path and not out.tokenizer_id
        lib.adamw_free(o)
        s.free()
    # the inference path reads the weights section of a checkpoint
    ws = ncmhip.WeightStore()
    assert ours.weights_load(ctypes.byref(ws), str(a).encode()) == 0
    assert same(read_store(ours, ws), trained)
    ours.weights_free(ctypes.byref(ws))
    for lib, (s, o) in zip(libs, ((s1, o1), (s2, o2))):
        lib.adamw_free(o)
        s.free()


def test_nck1_info_matches_reference(libs, tmp_path, capfd):
    ours, ref = libs
    spec = tensors_spec(6)
    (s1, o1), (s2, o2) = both_trained(libs, spec, [1.0] * 5, steps=1)
    path = tmp_path / "i.nckpt"
    assert save(ours, s1, o1, run_state(), path)[0] == 0
    libc = ctypes.CDLL(None)
    outs = []
    for lib in libs:
        capfd.readouterr()
        rc = lib.ckpt_info(str(path).encode())
        libc.fflush(None)
        outs.append((rc, capfd.readouterr().out))
    assert outs[0] == outs[1] and outs[0][0] == 0 and "status: valid" in outs[0][1]
    for lib, (s, o) in zip(libs, ((s1, o1), (s2, o2))):
        lib.adamw_free(o)
        s.free()


REFUSALS = {
    # case: (how the file or expectation changes, message fragment)
    "bitflip": ("flip", "checksum does not match"),
    "truncated": ("cut", "checksum does not match"),
    "tiny": ("tiny", "too small or too large"),
    "data_hash": ("ex:data_hash=1", "training data differ"),
    "rows": ("ex:n_rows=4999", "training data differ"),
    "conf": ("ex:conf_hash=2", "configuration hash differs"),
    "tokenizer": ("ex:tokenizer_id=b'llama'", "tokenizer 'gpt2' in the file"),
    "lr": ("ex:base_lr=1e-3", "schedule differs"),
    "wd": ("ex:wd=0.01", "optimizer section differs"),
    "pending": ("rs:accum_pending=2", "accumulation steps pending"),
    "garbage": ("garbage", "unexpected bytes"),
    "missing": ("missing", "cannot open"),
}


@pytest.mark.parametrize("case", sorted(REFUSALS))
def test_nck1_refusals_leave_state_untouched(libs, tmp_path, case):
    ours, ref = libs
    spec = tensors_spec(7)
    (s1, o1), (s2, o2) = both_trained(libs, spec, [1.0] * 5, steps=2)
    how, frag = REFUSALS[case]
    path = tmp_path / "c.nckpt"
    assert save(ours, s1, o1, run_state(), path)[0] == 0
    raw = bytearray(path.read_bytes())
    ex = expect()
    if how == "flip":
        raw[len(raw) // 2] ^= 0x10
    elif how == "cut":
        raw = raw[:-100]
    elif how == "tiny":
        raw = raw[:5]
    elif how == "garbage":
        body = bytes(raw[:-8]) + b"\x00" * 12
        raw = bytearray(body + struct.pack("<Q", fnv1a(body)))
    elif how.startswith("ex:"):
        k, v = how[3:].split("=")
        setattr(ex, k, eval(v))
    elif how.startswith("rs:"):  # a file that records pending accumulation (written by hand)
        off = 4 + 4 + 8 + 8 + 24 + 4
        raw[off:off + 4] = struct.pack("<i", 2)
        body = bytes(raw[:-8])
        raw = bytearray(body + struct.pack("<Q", fnv1a(body)))
    if how == "missing":
        path = tmp_path / "absent.nckpt"
    else:
        path.write_bytes(bytes(raw))
    # live state to protect: a second trained state
    (t1, p1), (t2, p2) = both_trained(libs, spec, [1.0] * 5, steps=1, seed=9)
    before = [(read_store(lib, t.ws), opt_state(lib, p)) for lib, (t, p) in zip(libs, ((t1, p1), (t2, p2)))]
    for k, (lib, t, p) in enumerate(((ours, t1, p1), (ref, t2, p2))):
        rc, err, _ = load(lib, t, p, ex, path)
        assert rc != 0
        if lib is ref:
            # the reference writes the weights before it checks the optimizer
            # section (ckpt.c:461-464), so only its refusal is compared
            continue
        assert frag in err, err
        after_w, (after_o, after_step) = read_store(lib, t.ws), opt_state(lib, p)
        assert same(after_w, before[k][0]) and after_step == before[k][1][1]
        for x, y in zip(after_o, before[k][1][0]):
            for u, w in zip(x, y):
                assert np.array_equal(u.view(np.uint32), w.view(np.uint32))
    for lib, (s, o) in zip(libs + libs, ((s1, o1), (s2, o2), (t1, p1), (t2, p2))):
        lib.adamw_free(o)
        s.free()


def test_nck1_save_refuses_pending_accumulation(libs, tmp_path):
    ours = libs[0]
    s = Store(ours, tensors_spec(8))
    o = make_opt(ours, s, [1.0] * 5)
    rc, err = save(ours, s, o, run_state(accum_pending=1), tmp_path / "p.nckpt")
    assert rc != 0 and "pending" in err and not os.listdir(tmp_path)
    ours.adamw_free(o)
    s.free()
