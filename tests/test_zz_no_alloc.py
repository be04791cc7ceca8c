"""uq_gemm_static, the GEMM entry point that allocates nothing, through the C ABI.

It runs uq_gemm's kernels on a fixed device array inside the library
(UQ_GEMM_SCRATCH_BYTES per GPU) instead of a workspace it allocates, so its
outputs must equal uq_gemm's bit for bit on the same inputs. Two calls in a
row, the second smaller, check that the array's leftover contents from the
first call do not leak into the second; a call whose workspace exceeds the
array is refused with UQ_ERR_ARG before anything is launched.
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import uq
import uq.synth as S
from helpers import assert_bitwise, assert_close, gemm_reference

pytestmark = pytest.mark.gpu


def _run(fn, W, X, N):
    M = X.shape[0]
    dx, dy = uq.DeviceArray.from_numpy(np.ascontiguousarray(X, np.float32)), uq.DeviceArray(4 * M * N)
    dy.upload(np.full(M * N, np.nan, np.float32))
    fn(W, M, dx, dy)
    uq.synchronize()
    return dy.download(np.float32, M * N).reshape(M, N)


@pytest.mark.parametrize("dtype,K,N,Ms", [(S.Q4_K, 4096, 12288, (512, 128)), (S.Q6_K, 12288, 4096, (300, 20)),
                                          (S.Q8_0, 4096, 1000, (70, 3))])
def test_gemm_static_equals_gemm_on_two_calls_the_second_smaller(dtype, K, N, Ms):
    w = S.weights(dtype, N, K, seed=S.seed_for(3) + dtype)
    W = uq.Weights(w, dtype, K, N)
    for i, M in enumerate(Ms):
        X = S.activations(K, seed=100 * i + M, rows=M).reshape(M, K)
        got = _run(uq.gemm_static, W, X, N)
        ref = _run(uq.gemm, W, X, N)
        assert_bitwise(got, ref, f"gemm_static vs gemm, call {i} M={M}")
        R = gemm_reference(dtype, w, N, K, X[:4])
        for m in range(len(R)):
            assert_close(got[m], R[m], what=f"gemm_static call {i} row {m}")
    W.free()


def test_gemm_static_refuses_a_workspace_beyond_the_array():
    K, N, M = 4096, 256, 4096  # activation planes alone: 2 * 4096 * 4096 * 2 bytes > 64 MiB
    W = uq.Weights(S.weights(S.Q4_K, N, K, seed=1), S.Q4_K, K, N)
    dx, dy = uq.DeviceArray(4 * M * K), uq.DeviceArray(4 * M * N)
    dy.upload(np.full(M * N, 7.0, np.float32))
    with pytest.raises(uq.UqError) as e:
        uq.gemm_static(W, M, dx, dy)
    assert e.value.kind == "ARG" and "exceeds" in str(e.value)
    uq.synchronize()
    assert np.all(dy.download(np.float32, M * N) == 7.0), "nothing written after the refusal"
    W.free()


@pytest.mark.parametrize("dtype,K,N,M", [(S.F32, 4096, 64, 4096), (S.Q4_K, 4096, 300, 1)])
def test_gemm_static_needs_no_workspace_for_gemv_calls(dtype, K, N, M):
    """Calls that run as GEMVs (F32 weights, one row) need no workspace:
    uq_gemm_static takes them even where the activation planes of an MFMA
    call (4*M*K bytes, 32 MiB here for F32; 64 MiB at M = 4096) would exceed the fixed array,
    with uq_gemm's bits."""
    W = uq.Weights(S.weights(dtype, N, K, seed=3), dtype, K, N)
    X = S.activations(K, seed=4, rows=M).reshape(M, K)
    got = _run(uq.gemm_static, W, X, N)
    ref = _run(uq.gemm, W, X, N)
    assert_bitwise(got, ref, f"gemm_static vs gemm dtype {dtype} M={M}")
    W.free()


def test_gemm_static_first_call_captured_in_a_graph():
    """The first uq_gemm_static call of a fresh process (its one-time set-up
    inside the capture), replayed twice from a HIP graph: every replay equals
    an eager uq_gemm bit for bit (tests/capture_child.py, a child process)."""
    child = os.path.join(os.path.dirname(os.path.abspath(__file__)), "capture_child.py")
    r = subprocess.run([sys.executable, "-u", child], capture_output=True, text=True, timeout=300)
    print(r.stderr[-2000:], flush=True)
    assert r.returncode == 0, f"child exit {r.returncode}: {r.stdout[-2000:]} {r.stderr[-2000:]}"
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["ok"], out
