"""Config 5 at its workload (12 layers, d 768, 12 heads, vocab 4096, 32 x 512
tokens): the device tape's forward, mean cross-entropy and backward, checked
against the CPU:

- the whole step: loss and all 148 parameter gradients against the CPU
  result of the same step (tests/golden/gpt2_c5_grads.npz, written by
  tests/golden/gen_gpt2_c5.py with the oracle, which is bit-equal to the
  reference's train_gpt2_forward + t_ce + tape_backward_host,
  train_gpt2.c:42-147, train_tape.c:442-481, 636-1051): per tensor the L2
  norm, four +-1 checksums (each moved by every element's error) and 64
  sampled entries, relative L2 within 1e-3 (the north star's gradient bar);
- the step composed here from the exported ncm_t_* recorders (as
  train_gpt2.c:42-147 does) gives the same loss and the same gradients, bit
  for bit, as the library's ncm_gpt2_forward driver;
- per op at the full R = 16384 rows, each fed the device's own upstream
  gradient and checked against the oracle on sampled slices (exact by the
  row/column separability of every reduction): c_fc and mlp.c_proj of the
  first and last block (dW and db rows over all 16384 rows, dx rows; for
  c_proj passed back through the GELU, which its dX GEMM does in the
  epilogue); SDPA backward (causal, T = 512) on sampled (batch, head) slices;
  softmax cross-entropy (the loss over all rows, dlogits on sampled rows);
  the tied head's dx rows and ln_f's dw, db (over all rows) and dx rows.

Bars are scale-aware per checked tensor (the mean over 16384 rows makes
these gradients 1e-6 to 1e-9 in size, so an absolute bar could not fail):
||got - ref||_2 <= 1e-4 ||ref||_2 and max |got - ref| <= 1e-4 max |ref|, with
ref not all zero; the loss to 1e-5 relative."""
import ctypes
import os

import numpy as np
import pytest

import model_data as MD
import ncmhip
import oracle as O
from conftest import GOLDEN

pytestmark = pytest.mark.gpu
D = ncmhip.DeviceBuffer

L, C, H, V, NPOS, B, T = 12, 768, 12, 4096, 512, 32, 512
HD, R, I = C // H, B * T, 4 * C


@pytest.fixture(scope="module", autouse=True)
def device():
    ncmhip.init(0)
    ncmhip.load().arena_init(24 << 30)
    ncmhip.check()
    print("[gpu] config-5 full-size gradient tests on device 0", flush=True)


class PMap(ctypes.Structure):
    _fields_ = [("params", ctypes.c_void_p), ("grads", ctypes.c_void_p), ("sizes", ctypes.c_void_p),
                ("n", ctypes.c_int)]

    def __init__(self, p, g, s, n):
        self._keep = (p, g, s)
        super().__init__(ctypes.cast(p, ctypes.c_void_p), ctypes.cast(g, ctypes.c_void_p),
                         ctypes.cast(s, ctypes.c_void_p), n)


def host(ptr, shape, dtype=np.float32):
    out = np.empty(shape, dtype)
    ncmhip.load().mem_d2h(out.ctypes.data, ptr, out.nbytes)
    ncmhip.check()
    return out


def weights():
    return MD.gpt2_c5_weights()


def close(got, ref, what, bar=1e-4):
    """Scale-aware closeness of one checked tensor: relative L2 and max
    error against the largest reference value, both <= bar; returns the
    relative L2 error."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    scale = float(np.max(np.abs(ref)))
    assert scale > 0, (what, "reference is all zero")
    d = got - ref
    rel = float(np.sqrt(np.sum(d * d) / np.sum(ref * ref)))
    mx = float(np.max(np.abs(d))) / scale
    print(f"[c5] {what}: rel-L2 {rel:.2e}, max/max|ref| {mx:.2e}")
    assert rel <= bar and mx <= bar, (what, rel, mx)
    return rel


@pytest.fixture(scope="module")
def step():
    """One composed step (activations kept) and one driver step."""
    lib = ncmhip.load()
    params, ids, tgt = weights()
    P = [D.from_numpy(p) for p in params]
    sizes = (ctypes.c_int64 * len(P))(*[p.size for p in params])
    A = lambda n: lib.arena_alloc(n)  # noqa: E731

    # -- the library's driver --
    G1 = [D.from_numpy(np.zeros_like(p)) for p in params]
    t1 = lib.ncm_tape_new()
    lib.arena_reset()
    cfg = ncmhip.Gpt2Config(L, C, H, V, NPOS)
    logits1 = lib.ncm_gpt2_forward(t1, ctypes.byref(cfg), ncmhip.ptr_array(P), ids.ctypes.data, B, T)
    ncmhip.check()
    loss1 = D.empty(1)
    lib.ncm_t_ce(t1, logits1, tgt.ctypes.data, None, loss1.ptr, None, R, V, 1.0)
    lib.ncm_tape_backward(t1, ctypes.byref(PMap(ncmhip.ptr_array(P), ncmhip.ptr_array(G1), sizes, len(P))))
    ncmhip.check()
    g1 = [g.numpy() for g in G1]
    l1 = float(loss1.numpy()[0])
    lib.ncm_tape_free(t1)
    del G1
    print("[gpu] driver step done", flush=True)

    # -- the same step from the recorders, keeping pointers --
    lib.arena_reset()
    tp = lib.ncm_tape_new()
    G = [D.from_numpy(np.zeros_like(p)) for p in params]
    pos = np.tile(np.arange(T, dtype=np.int32), B)
    xe, pe, h = A(R * C), A(R * C), A(R * C)
    lib.ncm_t_embed(tp, P[0].ptr, ids.ctypes.data, V, xe, R, C)
    lib.ncm_t_embed(tp, P[1].ptr, pos.ctypes.data, NPOS, pe, R, C)
    lib.ncm_t_add(tp, xe, pe, h, R * C)
    mask_h = np.where(np.arange(T)[None, :] <= np.arange(T)[:, None], 0.0, -1e9).astype(np.float32)
    mask = D.from_numpy(mask_h)
    keep = {}
    for li in range(L):
        w = [P[2 + 12 * li + j].ptr for j in range(12)]
        ln, qkv, qq, kk, vv, ctx = A(R * C), A(R * 3 * C), A(R * C), A(R * C), A(R * C), A(R * C)
        mo, ao, x1, mn, mm, m2, mlpo, out = (A(R * C), A(R * C), A(R * C), A(R * C), A(R * I), A(R * I),
                                             A(R * C), A(R * C))
        lib.ncm_t_layernorm_eps(tp, h, w[0], w[1], ln, R, C, 1e-5)
        lib.ncm_t_linear(tp, ln, w[2], w[3], qkv, R, 3 * C, C)
        lib.ncm_t_qkvsplit(tp, qkv, qq, kk, vv, B, T, C, H, HD, H, 1)
        lib.ncm_t_sdpa(tp, qq, kk, vv, mask.ptr, ctx, B, H, H, T, T, HD)
        lib.ncm_t_headmerge(tp, ctx, mo, B, T, C, H, HD)
        lib.ncm_t_linear(tp, mo, w[4], w[5], ao, R, C, C)
        lib.ncm_t_add(tp, h, ao, x1, R * C)
        lib.ncm_t_layernorm_eps(tp, x1, w[6], w[7], mn, R, C, 1e-5)
        lib.ncm_t_linear(tp, mn, w[8], w[9], mm, R, I, C)
        lib.ncm_t_gelu_tanh(tp, mm, m2, R * I)
        lib.ncm_t_linear(tp, m2, w[10], w[11], mlpo, R, C, I)
        lib.ncm_t_add(tp, x1, mlpo, out, R * C)
        keep[li] = dict(qkv=qkv, qq=qq, kk=kk, vv=vv, ctx=ctx, mn=mn, mm=mm, m2=m2, mlpo=mlpo)
        h = out
    ncmhip.check()
    n = len(P)
    lnf, logits = A(R * C), A(R * V)
    lib.ncm_t_layernorm_eps(tp, h, P[n - 2].ptr, P[n - 1].ptr, lnf, R, C, 1e-5)
    lib.ncm_t_linear(tp, lnf, P[0].ptr, None, logits, R, V, C)
    loss = D.empty(1)
    lib.ncm_t_ce(tp, logits, tgt.ctypes.data, None, loss.ptr, None, R, V, 1.0)
    lib.ncm_tape_backward(tp, ctypes.byref(PMap(ncmhip.ptr_array(P), ncmhip.ptr_array(G), sizes, len(P))))
    ncmhip.check()
    print("[gpu] composed step done", flush=True)
    st = dict(lib=lib, tp=tp, params=params, ids=ids, tgt=tgt, G=G, g1=g1, l1=l1, loss=float(loss.numpy()[0]),
              keep=keep, h=h, lnf=lnf, logits=logits, grad=lambda p: lib.ncm_tape_grad(tp, p))
    yield st
    lib.ncm_tape_free(tp)


def test_driver_equals_composed_step(step):
    assert step["loss"] == step["l1"]
    for i, (g, r) in enumerate(zip(step["G"], step["g1"])):
        assert np.array_equal(g.numpy().view(np.uint32), r.view(np.uint32)), i


def sample(n, k, seed):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, n - 1], rng.choice(n, k, replace=False)]))


@pytest.mark.parametrize("li", [0, L - 1])
def test_mlp_linears_full_rows(step, li):
    params, G, keep = step["params"], step["G"], step["keep"][li]
    for which, (xkey, ykey, wi, K, N) in {"c_fc": ("mn", "mm", 8, C, I), "c_proj": ("m2", "mlpo", 10, I, C)}.items():
        x = host(keep[xkey], (R, K))
        dy = host(step["grad"](keep[ykey]), (R, N))
        W = params[2 + 12 * li + wi]
        ms = sample(N, 30, li * 7 + wi)
        _, dW, db = O.linear_bwd(x, W[ms], dy[:, ms], want=("dW", "db"))   # sums over all 16384 rows
        gW, gb = G[2 + 12 * li + wi].numpy(), G[3 + 12 * li + wi].numpy()
        close(gW[ms], dW, f"layer {li} {which} dW")
        close(gb[ms], db, f"layer {li} {which} db")
        rs = sample(R, 30, li * 11 + wi)
        dx, _, _ = O.linear_bwd(x[rs], W, dy[rs], want=("dx",))
        if which == "c_fc":   # mn feeds only c_fc: its gradient is this product's dx
            got_dx = host(step["grad"](keep[xkey]), (R, K))[rs]
        else:
            # m2 = gelu_tanh(mm) feeds only c_proj, so c_proj's dX GEMM applies
            # the GELU backward in its epilogue and m2's gradient is never
            # stored: check mm's gradient (mm feeds only the GELU)
            dx = O.act_bwd("gelu_tanh", host(keep["mm"], (R, I))[rs], dx)
            got_dx = host(step["grad"](keep["mm"]), (R, I))[rs]
        close(got_dx, dx, f"layer {li} {which} dx")


@pytest.mark.parametrize("li", [0, L - 1])
def test_sdpa_backward_t512_slices(step, li):
    keep = step["keep"][li]
    q, k, v = (host(keep[n], (B, H, T, HD)) for n in ("qq", "kk", "vv"))
    dO = host(step["grad"](keep["ctx"]), (B, H, T, HD))
    # q, k and v feed only the attention, and the split that made them stands
    # right before it: the attention's backward writes their gradients straight
    # into the qkv rows' gradient [R][3C] (q | k | v, head h at columns 64 h)
    gqkv = host(step["grad"](keep["qkv"]), (B, T, 3, H, HD))
    gq, gk, gv = (np.ascontiguousarray(gqkv[:, :, j].transpose(0, 2, 1, 3)) for j in range(3))
    mask = np.where(np.arange(T)[None, :] <= np.arange(T)[:, None], 0.0, -1e9).astype(np.float32)
    for b, hh in ((0, 0), (B - 1, H - 1), (13, 5)):
        sl = np.s_[b:b + 1, hh:hh + 1]
        Pm = O.sdpa_probs(q[sl], k[sl], mask)
        dq, dk, dv = O.sdpa_bwd(q[sl], k[sl], v[sl], Pm, dO[sl])
        for name, got, ref in (("dq", gq[sl], dq), ("dk", gk[sl], dk), ("dv", gv[sl], dv)):
            close(got, ref, f"layer {li} sdpa ({b},{hh}) {name}")


def test_cross_entropy_full_rows(step):
    logits = host(step["logits"], (R, V))
    tgt = step["tgt"].reshape(-1)
    loss, probs, cnt = O.ce_fwd(logits, tgt)
    assert cnt == R
    assert abs(step["loss"] - loss) <= 1e-5 * abs(loss)
    rs = sample(R, 64, 3)
    dl = O.ce_bwd(probs[rs], tgt[rs], None, 1.0 / cnt)
    got = host(step["grad"](step["logits"]), (R, V))[rs]
    close(got, dl, "dlogits")


def test_head_and_final_norm_full_rows(step):
    params, G = step["params"], step["G"]
    n = len(params)
    dlog = host(step["grad"](step["logits"]), (R, V))
    rs = sample(R, 30, 5)
    dx, _, _ = O.linear_bwd(np.zeros((rs.size, C), np.float32), params[0], dlog[rs], want=("dx",))
    dlnf = host(step["grad"](step["lnf"]), (R, C))
    close(dlnf[rs], dx, "head dx")
    h = host(step["h"], (R, C))
    dxn, dw, db = O.layernorm_bwd(h, params[n - 2], dlnf, eps=1e-5)      # dw, db over all rows
    close(G[n - 2].numpy(), dw, "ln_f dw")
    close(G[n - 1].numpy(), db, "ln_f db")
    gh = host(step["grad"](step["h"]), (R, C))
    close(gh[rs], dxn[rs], "ln_f dx")


FIXTURE = os.path.join(GOLDEN, "gpt2_c5_grads.npz")


@pytest.mark.skipif(not os.path.exists(FIXTURE), reason="tests/golden/gpt2_c5_grads.npz not generated")
def test_whole_step_gradients_match_cpu(step):
    """Every parameter gradient of the 12-layer step against the CPU's (the
    drift of 12 layers of fp32 MFMA arithmetic against the reference's fp64
    accumulations), relative L2 <= 1e-3 per tensor, estimated three ways:
    the norm, the +-1 checksums (sqrt of the mean squared checksum error is
    the error's L2 norm in expectation) and the sampled entries."""
    fx = np.load(FIXTURE, allow_pickle=False)
    ref_loss = float(fx["loss"])
    print(f"[c5] loss {step['l1']:.9g} against the CPU's {ref_loss:.9g}")
    assert abs(step["l1"] - ref_loss) <= 1e-5 * abs(ref_loss)
    worst = (0.0, None)
    for i, g in enumerate(step["g1"]):
        f = g.reshape(-1).astype(np.float64)
        nref = float(fx["norms"][i])
        assert nref > 0, i
        e_norm = abs(float(np.sqrt(np.dot(f, f))) - nref) / nref
        dp = np.array([np.dot(f, MD.grad_probe_signs(f.size, 7000 + 10 * i + j)) for j in range(fx["probes"].shape[1])])
        e_probe = float(np.sqrt(np.mean((dp - fx["probes"][i]) ** 2))) / nref
        sv = fx["val"][i].astype(np.float64)
        ds = f[fx["idx"][i]] - sv
        e_samp = float(np.sqrt(np.sum(ds * ds) / max(np.sum(sv * sv), 1e-300)))
        e = max(e_norm, e_probe, e_samp)
        if e > worst[0]:
            worst = (e, i)
        assert e_norm <= 1e-3 and e_probe <= 1e-3 and e_samp <= 1e-3, (i, e_norm, e_probe, e_samp)
    print(f"[c5] worst relative gradient error over {len(step['g1'])} tensors: {worst[0]:.2e} (tensor {worst[1]})")
