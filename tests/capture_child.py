"""Child process for tests/test_zz_no_alloc.py: the first uq_gemm_static call of
a fresh process, captured into a HIP graph.

The first call on a device looks up the fixed workspace's address and raises
the GEMM kernels' LDS limits; here those set-up calls run while the stream is
being captured. The graph is replayed twice and each replay's output is
compared bit for bit with an eager uq_gemm of the same inputs.

    python tests/capture_child.py   (prints one JSON line; exit 0 when all replays match)
"""
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path[:0] = [ROOT, os.path.join(ROOT, "unltd-inference_amd")]

import numpy as np  # noqa: E402

import bench  # noqa: E402
import uq  # noqa: E402
import uq.synth as S  # noqa: E402

# (dtype, K, N, M): a split-K small-M call (the loader-wave kernel and the
# partial-tile reduction) and a 128-row tile call
CASES = [(S.Q4_K, 4096, 2048, 8), (S.Q4_K, 4096, 1536, 200)]


def main():
    hip = bench.Hip()
    s = hip.stream()
    staged = []
    for dt, K, N, M in CASES:
        W = uq.Weights(S.weights(dt, N, K, seed=K + N + M), dt, K, N)
        X = S.activations(K, seed=M, rows=M).reshape(M, K)
        dx, dy = uq.DeviceArray.from_numpy(X), uq.DeviceArray(4 * M * N)
        staged.append((W, M, N, dx, dy))
    hip.sync()
    print("inputs staged; capturing the first uq_gemm_static calls", file=sys.stderr, flush=True)
    g = hip.capture(s, lambda: [uq.gemm_static(W, M, dx, dy, s) for W, M, N, dx, dy in staged])
    res = {}
    replays = []
    for rep in range(2):
        for _, M, N, _, dy in staged:
            dy.upload(np.full(M * N, np.nan, np.float32))
        hip.launch_graph(g, s)
        hip.sync()
        replays.append([dy.download(np.float32, M * N) for _, M, N, _, dy in staged])
    ok = True
    for i, (W, M, N, dx, dy) in enumerate(staged):
        ref = uq.DeviceArray(4 * M * N)
        uq.gemm(W, M, dx, ref, s)
        hip.sync()
        r = ref.download(np.float32, M * N)
        same = [bool(np.array_equal(rp[i].view(np.uint32), r.view(np.uint32))) for rp in replays]
        res[f"case{i}_M{M}_N{N}"] = same
        ok = ok and all(same) and bool(np.all(np.isfinite(r)))
    print(json.dumps({"replays_equal_eager": res, "ok": ok}), flush=True)
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
