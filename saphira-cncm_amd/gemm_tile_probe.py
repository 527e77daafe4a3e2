"""Times the linear layer's forward and dX products on each forced tile
mode (ncm_hip_set_gemm_tiles: 64 = 64 x 64, 128 = 128 x 128, 0 = the
library's choice) for a list of shapes, operands rotated through three
copies, and prints the per-call time and TFLOP/s of each: the measurements
the GEMM cost model in csrc/linear.c is fitted to.  Before timing, each
mode's forward, dX and dW + db are checked against numpy on integer-valued
operands (exact in fp32).

    python3 saphira-cncm_amd/gemm_tile_probe.py [--modes 64,128] [M,K,N ...]

Needs a GPU; the library must be built (__graft_entry__.build())."""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import ncmhip  # noqa: E402

SHAPES = [(8192, 256, 1024), (8192, 1024, 1024), (8192, 2048, 1024), (8192, 4096, 1024),
          (4096, 768, 3072), (4096, 896, 4864), (4096, 3072, 768), (4096, 4096, 4096),
          (16384, 768, 2304), (16384, 768, 3072), (16384, 3072, 768)]
COPIES = 3


def per_call_ms(fn, reps=12, warm=3):
    for i in range(warm):
        fn(i)
    ncmhip.sync()
    e0, e1 = ncmhip.Event(), ncmhip.Event()
    e0.record()
    for i in range(reps):
        fn(i)
    e1.record()
    e1.synchronize()
    return e0.elapsed_ms(e1) / reps


def check(lib, modes):
    D = ncmhip.DeviceBuffer
    rng = np.random.default_rng(1)
    for M, K, N in ((300, 200, 260), (256, 96, 192), (1000, 768, 2304)):
        x = rng.integers(-3, 4, (M, K)).astype(np.float32)
        W = rng.integers(-3, 4, (N, K)).astype(np.float32)
        b = rng.integers(-3, 4, N).astype(np.float32)
        dy = rng.integers(-3, 4, (M, N)).astype(np.float32)
        for mode in modes:
            lib.ncm_hip_set_gemm_tiles(mode)
            y, dx, dW, db = D.empty((M, N)), D.from_numpy(np.ones((M, K), np.float32)), \
                D.from_numpy(np.ones((N, K), np.float32)), D.from_numpy(np.ones(N, np.float32))
            ncmhip.linear_fwd(D.from_numpy(x), D.from_numpy(W), D.from_numpy(b), y, M, N, K)
            ncmhip.linear_bwd(D.from_numpy(x), D.from_numpy(W), D.from_numpy(dy), dx, dW, db, M, N, K)
            ok = (np.array_equal(y.numpy(), x @ W.T + b) and np.array_equal(dx.numpy(), 1 + dy @ W)
                  and np.array_equal(dW.numpy(), 1 + dy.T @ x) and np.array_equal(db.numpy(), 1 + dy.sum(0)))
            print(f"check {M}x{K}->{N} tiles {mode}: {'exact' if ok else 'MISMATCH'}", flush=True)
            if not ok:
                raise SystemExit(1)
    lib.ncm_hip_set_gemm_tiles(0)


def main(shapes, modes):
    ncmhip.init(0)
    lib = ncmhip.load()
    check(lib, modes)
    D = ncmhip.DeviceBuffer
    rng = np.random.default_rng(0)
    print("M K N | tiles: forward us TFLOP/s, dX us TFLOP/s", flush=True)
    for M, K, N in shapes:
        xs = [D.from_numpy(rng.standard_normal((M, K), dtype=np.float32)) for _ in range(COPIES)]
        Ws = [D.from_numpy(rng.standard_normal((N, K), dtype=np.float32) / np.float32(np.sqrt(K)))
              for _ in range(COPIES)]
        ys = [D.empty((M, N)) for _ in range(COPIES)]
        dys = [D.from_numpy(rng.standard_normal((M, N), dtype=np.float32)) for _ in range(COPIES)]
        dxs = [D.empty((M, K)) for _ in range(COPIES)]
        flop = 2.0 * M * N * K
        out = []
        for mode in modes:
            lib.ncm_hip_set_gemm_tiles(mode)
            tf = per_call_ms(lambda i: ncmhip.linear_fwd(xs[i % COPIES], Ws[i % COPIES], None, ys[i % COPIES],
                                                         M, N, K))
            tb = per_call_ms(lambda i: ncmhip.linear_bwd(xs[i % COPIES], Ws[i % COPIES], dys[i % COPIES],
                                                         dxs[i % COPIES], None, None, M, N, K))
            out.append(f"{mode}: {tf * 1e3:7.1f} {flop / tf / 1e9:6.1f}, {tb * 1e3:7.1f} {flop / tb / 1e9:6.1f}")
        lib.ncm_hip_set_gemm_tiles(0)
        print(f"{M} {K} {N} | " + " | ".join(out), flush=True)


if __name__ == "__main__":
    argv = sys.argv[1:]
    modes = (64, 128)
    if argv[:1] == ["--modes"]:
        modes = tuple(int(v) for v in argv[1].split(","))
        argv = argv[2:]
    main([tuple(int(v) for v in a.split(",")) for a in argv] or SHAPES, modes)
