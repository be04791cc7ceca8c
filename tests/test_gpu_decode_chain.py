"""The decode step as the benchmark runs it: every quantized linear layer of
the synthetic hybrid 9B (32 layers, 24 GatedDeltaNet + 8 attention, FFN
12288, Q6_K head 152064; bench.py's DecodeStep) captured as one HIP graph.

The graph is replayed twice with an eager run of the same launches between
the replays: all three leave the same bits in every buffer. Every launch's
output is then checked against the oracle applied to that launch's input
as it sits on the device:
  * gemv_quant semantics: each projection within |y - r| <= 1e-4 + 1e-3 |r|;
    h of the fused FFN within that tolerance propagated through SwiGLU;
  * gemv_quant_q8k semantics (the reference forward's numerics,
    qwen35_forward.rs:365-401, :735-765, min_forward.rs:248-264): every
    projection, g, u and the down projection bit for bit; h within 2 ulp of
    the oracle's swiglu of the device's g and u (the reference's expf is the
    platform libm's, the device evaluates exp in f64 and rounds once).
"""
import os
import sys

import numpy as np
import pytest

import oracle as O
from helpers import assert_bitwise, assert_close, swiglu_bound

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def step():
    import bench
    log("decode chain: uploading 4.6 GB of weights")
    st = bench.DecodeStep()
    yield bench, st
    st.free()
    st.head.free()


def snapshot(st):
    out = []
    for L in st.layers:
        out.append({k: L["buf"][k].download(np.float32, n) for k, n in L["size"].items()})
    return out, st.logits.download(np.float32, 152064)


def same_bits(a, b, what):
    (la, ha), (lb, hb) = a, b
    for il, (x, y) in enumerate(zip(la, lb)):
        for k in x:
            assert_bitwise(x[k], y[k], f"{what} layer {il} {k}")
    assert_bitwise(ha, hb, f"{what} logits")


def oracle_gemv(q8k, w, x, K, N, dt):
    r = np.zeros(N, np.float32)
    (O.gemv_quant_q8k if q8k else O.gemv_quant)(r, x, w, K, N, dt, nthreads=NT)
    return r


@pytest.mark.parametrize("q8k", [False, True], ids=["gemv_quant", "gemv_quant_q8k"])
def test_decode_chain_graph_every_launch_against_oracle(step, q8k):
    bench, st = step
    hip = bench.Hip()
    s = hip.stream()
    graph = hip.capture(s, lambda: st.chain(s, q8k=q8k))
    hip.launch_graph(graph, s)
    hip.sync()
    first = snapshot(st)
    st.chain(s, q8k=q8k)  # the same launches eagerly
    hip.sync()
    same_bits(first, snapshot(st), "eager vs graph replay 1")
    hip.launch_graph(graph, s)
    hip.sync()
    same_bits(first, snapshot(st), "graph replay 2 vs replay 1")
    log(f"decode chain q8k={q8k}: replays agree; checking {st.launches()} launches against the oracle")

    layers, logits = first
    x = st.x_host
    for il, (L, B) in enumerate(zip(st.layers, layers)):
        shapes = {name: (dt, K, N) for name, dt, K, N in L["shape"]}

        def proj(name, inp, got):
            dt, K, N = shapes[name]
            r = oracle_gemv(q8k, st.host[(dt, K, N)], inp, K, N, dt)
            if q8k:
                assert_bitwise(got, r, f"layer {il} {name}")
            else:
                assert_close(got, r, what=f"layer {il} {name}")

        if L["attn"]:
            proj("attn_q", x, B["a"])
            proj("attn_k", x, B["c"])
            proj("attn_v", x, B["d"])
            proj("attn_output", B["a"][:4096], B["o"])
        else:
            proj("attn_qkv", x, B["a"])
            proj("attn_gate", x, B["b"])
            proj("ssm_beta", x, B["e"])
            proj("ssm_alpha", x, B["f"])
            proj("ssm_out", B["b"], B["o"])
        dtg, Kg, Ng = shapes["ffn_gate"]
        rg = oracle_gemv(q8k, st.host[(dtg, Kg, Ng)], B["o"], Kg, Ng, dtg)
        ru = oracle_gemv(q8k, st.host[shapes["ffn_up"]], B["o"], Kg, Ng, dtg)
        if q8k:
            assert_bitwise(B["g"], rg, f"layer {il} ffn_gate")
            assert_bitwise(B["u"], ru, f"layer {il} ffn_up")
            sw = O.swiglu(B["g"], B["u"])
            ulp = np.abs(B["h"].view(np.int32).astype(np.int64) - sw.view(np.int32).astype(np.int64))
            assert int(ulp.max()) <= 2, f"layer {il} swiglu ulp {int(ulp.max())}"
        else:
            rh, bound = swiglu_bound(rg, ru)
            assert np.all(np.abs(B["h"].astype(np.float64) - rh) <= bound), f"layer {il} h"
        proj("ffn_down", B["h"], B["y"])
    head_host = st.head_host
    r = oracle_gemv(q8k, head_host, x, 4096, 152064, O.Q6_K)
    if q8k:
        assert_bitwise(logits, r, "head logits")
    else:
        assert_close(logits, r, what="head logits")
