"""Benchmark of the quantized linear-layer path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]

Headline workload (one "step" = one pass over one batch):
    Q6_K output-projection GEMV, 152064 x 4096 (510,935,040 weight bytes),
    gemv_quant semantics, weights and activations resident in HBM.
    value = algorithmic bytes (weights + 4K + 4N) per step / wall time per
    step, in GB/s; roofline.achieved uses HIP-event kernel time.
Secondary workloads (reported under "extra", not the headline):
    Q4_K GEMV 4096 x 4096 (rotated over 64 copies so the 256 MB MALL cannot
    serve it), fused FFN gate/up Q4_K 12288 x 4096 + SwiGLU + down Q6_K
    4096 x 12288 and a Q8_0 4096 x 4096 projection (rotated), the Q4_K prefill
    GEMM N=12288 K=4096 over M in {1, 8, 32, 128, 512}, bit-exact
    gemv_quant_q8k on the head, and the decode step of a synthetic 9B hybrid
    (all quantized linear layers back-to-back, replayed as one HIP graph).
cpu_baseline: the CPU oracle (a C restatement of the reference's scalar
kernels) on the same head weights, timed on this host.
Data are synthetic (seeded random GGUF blocks, N(0,1) activations).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import platform
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "unltd-inference_amd")]

import uq  # noqa: E402
import uq.synth as S  # noqa: E402

METRIC = "Q4_K/Q6_K GEMV achieved HBM GB/s (% of peak); decode-step linear-layer tok/s"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
PROFILES = os.path.join(ROOT, "profiles")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ----------------------------------------------------------- HIP plumbing
class Hip:
    """HIP runtime calls the timing needs (events, streams, graphs)."""

    def __init__(self):
        uq.lib()  # loads libamdhip64 into the process
        self.h = C.CDLL("libamdhip64.so")
        P = C.c_void_p
        self.h.hipEventCreate.argtypes = [C.POINTER(P)]
        self.h.hipEventRecord.argtypes = [P, P]
        self.h.hipEventSynchronize.argtypes = [P]
        self.h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), P, P]
        self.h.hipStreamCreate.argtypes = [C.POINTER(P)]
        self.h.hipStreamSynchronize.argtypes = [P]
        self.h.hipStreamBeginCapture.argtypes = [P, C.c_int]
        self.h.hipStreamEndCapture.argtypes = [P, C.POINTER(P)]
        self.h.hipGraphInstantiate.argtypes = [C.POINTER(P), P, P, P, C.c_size_t]
        self.h.hipGraphLaunch.argtypes = [P, P]

    def ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed: {rc}")

    def event(self):
        e = C.c_void_p()
        self.ok(self.h.hipEventCreate(C.byref(e)), "hipEventCreate")
        return e

    def stream(self):
        s = C.c_void_p()
        self.ok(self.h.hipStreamCreate(C.byref(s)), "hipStreamCreate")
        return s

    def sync(self):
        self.ok(self.h.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def record(self, e, s=None):
        self.ok(self.h.hipEventRecord(e, s), "hipEventRecord")

    def elapsed_ms(self, a, b):
        self.ok(self.h.hipEventSynchronize(b), "hipEventSynchronize")
        ms = C.c_float()
        self.ok(self.h.hipEventElapsedTime(C.byref(ms), a, b), "hipEventElapsedTime")
        return ms.value

    def capture(self, s, fn):
        self.ok(self.h.hipStreamBeginCapture(s, 0), "hipStreamBeginCapture")
        fn()
        g = C.c_void_p()
        self.ok(self.h.hipStreamEndCapture(s, C.byref(g)), "hipStreamEndCapture")
        ge = C.c_void_p()
        self.ok(self.h.hipGraphInstantiate(C.byref(ge), g, None, None, 0), "hipGraphInstantiate")
        return ge

    def launch_graph(self, ge, s):
        self.ok(self.h.hipGraphLaunch(ge, s), "hipGraphLaunch")


def timed(hip, fn, steps, warmup, stream=None):
    """Run warmup untimed steps, then exactly `steps` timed ones bracketed by
    device synchronisation; returns (wall_s, event_ms) for the whole region."""
    for _ in range(warmup):
        fn()
    hip.sync()
    e0, e1 = hip.event(), hip.event()
    t0 = time.perf_counter()
    hip.record(e0, stream)
    for _ in range(steps):
        fn()
    hip.record(e1, stream)
    hip.sync()
    wall = time.perf_counter() - t0
    return wall, hip.elapsed_ms(e0, e1)


def gemv_bytes(dtype, K, N):
    return S.row_bytes(dtype, K) * N + 4 * K + 4 * N


# ----------------------------------------------------------- workloads
def bench_head(hip, steps, warmup):
    K, N = 4096, 152064
    log("head: generating Q6_K 152064 x 4096")
    w = S.weights(S.Q6_K, N, K, seed=S.seed_for(1))
    x = S.activations(K, seed=S.seed_for(1))
    W = uq.Weights(w, uq.DType.Q6K, K, N)
    dx, dy = uq.DeviceArray.from_numpy(x), uq.DeviceArray(4 * N)
    nbytes = gemv_bytes(S.Q6_K, K, N)
    s = hip.stream()  # events are recorded on the stream the kernels run on
    wall, ev = timed(hip, lambda: uq.gemv(W, dx, dy, s), steps, warmup, s)
    res = {"bytes": nbytes, "wall_s": wall, "event_ms": ev, "steps": steps,
           "gbs_wall": nbytes * steps / wall / 1e9, "gbs_event": nbytes * steps / (ev * 1e-3) / 1e9,
           "us_per_call": ev * 1e3 / steps}
    # the integer-heavy q8k kernel runs 10-25% slower for its first several
    # ms after the memory-bound head (the shader clock settles; inside the
    # decode chain it takes 94 us): timed after 200 warmup calls (~25 ms)
    wall8, ev8 = timed(hip, lambda: uq.gemv_q8k(W, dx, dy, s), steps, max(warmup, 200), s)
    res["q8k"] = {"us_per_call": ev8 * 1e3 / steps, "gbs_event": nbytes * steps / (ev8 * 1e-3) / 1e9}
    return res, w, x, W


def rotated(hip, make_step, ncopies, steps, warmup):
    wall, ev = timed(hip, make_step, steps * ncopies, warmup * ncopies)
    return wall, ev


def bench_q4k_small(hip, steps, warmup):
    K, N, copies = 4096, 4096, 64
    w = S.weights(S.Q4_K, N, K, seed=S.seed_for(0))
    x = S.activations(K, seed=S.seed_for(0))
    Ws = [uq.Weights(w, uq.DType.Q4K, K, N) for _ in range(copies)]
    dx, dy = uq.DeviceArray.from_numpy(x), uq.DeviceArray(4 * N)
    state = {"i": 0}

    def step():
        uq.gemv(Ws[state["i"] % copies], dx, dy)
        state["i"] += 1

    wall, ev = timed(hip, step, steps * copies, warmup)
    n = steps * copies
    nbytes = gemv_bytes(S.Q4_K, K, N)
    for W in Ws:
        W.free()
    return {"config": "Q4_K GEMV 4096x4096, 64 rotated copies (605 MB)", "bytes": nbytes,
            "us_per_call": ev * 1e3 / n, "gbs_event": nbytes * n / (ev * 1e-3) / 1e9,
            "gbs_wall": nbytes * n / wall / 1e9}


def bench_q4k_large(hip, steps, warmup):
    """The Q4_K streaming kernel at the head's shape (152064 x 4096, 350 MB):
    one launch long enough that its fixed cost is amortised."""
    K, N = 4096, 152064
    w = S.weights(S.Q4_K, N, K, seed=S.seed_for(0, 7))
    x = S.activations(K, seed=S.seed_for(0, 7))
    W = uq.Weights(w, uq.DType.Q4K, K, N)
    dx, dy = uq.DeviceArray.from_numpy(x), uq.DeviceArray(4 * N)
    s = hip.stream()
    wall, ev = timed(hip, lambda: uq.gemv(W, dx, dy, s), steps, warmup, s)
    nbytes = gemv_bytes(S.Q4_K, K, N)
    W.free()
    gbs = nbytes * steps / (ev * 1e-3) / 1e9
    return {"config": "Q4_K GEMV 152064x4096 (350 MB)", "bytes": nbytes, "us_per_call": ev * 1e3 / steps,
            "gbs_event": gbs, "frac_hbm_peak": gbs / HBM_PEAK_GBS, "gbs_wall": nbytes * steps / wall / 1e9}


def bench_ffn(hip, steps, warmup):
    n, nff, copies = 4096, 12288, 6
    g = S.weights(S.Q4_K, nff, n, seed=S.seed_for(2, 1))
    u = S.weights(S.Q4_K, nff, n, seed=S.seed_for(2, 2))
    d = S.weights(S.Q6_K, n, nff, seed=S.seed_for(2, 3))
    q = S.weights(S.Q8_0, n, n, seed=S.seed_for(2, 4))
    x = S.activations(n, seed=S.seed_for(2))
    sets = [(uq.Weights(g, uq.DType.Q4K, n, nff), uq.Weights(u, uq.DType.Q4K, n, nff),
             uq.Weights(d, uq.DType.Q6K, nff, n), uq.Weights(q, uq.DType.Q8_0, n, n)) for _ in range(copies)]
    dx, dh, dy, dq = (uq.DeviceArray.from_numpy(x), uq.DeviceArray(4 * nff), uq.DeviceArray(4 * n),
                      uq.DeviceArray(4 * n))
    state = {"i": 0}

    def step():
        G, U, D, Q = sets[state["i"] % copies]
        uq.ffn_swiglu(G, U, D, dx, dh, dy)
        uq.gemv(Q, dx, dq)
        state["i"] += 1

    wall, ev = timed(hip, step, steps * copies, warmup)
    k = steps * copies
    wbytes = 2 * g.size + d.size + q.size
    act = 4 * n + 2 * 4 * nff + 4 * n + 4 * n + 4 * n  # x, h written+read, y, q8_0 x and y
    for s in sets:
        for W in s:
            W.free()
    return {"config": "FFN gate/up Q4_K 12288x4096 + SwiGLU, down Q6_K 4096x12288, + Q8_0 4096x4096; "
                      "6 rotated copies (694 MB)",
            "weight_bytes": wbytes, "us_per_step": ev * 1e3 / k,
            "gbs_event": (wbytes + act) * k / (ev * 1e-3) / 1e9}


def bench_gemm(hip, steps, warmup):
    """Prefill GEMM M sweeps: Q4_K N=12288 K=4096 (the prefill workload), and
    the same sweep for Q6_K (N=4096, K=12288, an FFN down shape) and Q8_0
    (N=12288, K=4096). Timed with HIP events on the launch stream."""
    s = hip.stream()
    out = {}
    for dt, name, K, N in ((S.Q4_K, "q4k", 4096, 12288), (S.Q6_K, "q6k", 12288, 4096), (S.Q8_0, "q80", 4096, 12288)):
        w = S.weights(dt, N, K, seed=S.seed_for(3))
        W = uq.Weights(w, dt, K, N)
        X = S.activations(K, seed=S.seed_for(3), rows=512)
        dx, dy = uq.DeviceArray.from_numpy(X), uq.DeviceArray(4 * 512 * N)
        by_m = {}
        for M in (1, 8, 32, 128, 512):
            # the MFMA-heavy kernels run slower for their first few ms (the clock settles):
            # 50 warmup calls, then at least 10 timed ones
            st = max(10, steps // (1 if M < 128 else 2))
            wall, ev = timed(hip, lambda: uq.gemm(W, M, dx, dy, s), st, max(warmup, 50), s)
            t = ev * 1e-3 / st
            by_m[str(M)] = {"us": t * 1e6, "tflops": 2 * M * N * K / t / 1e12,
                            "frac_bf16_peak": 2 * M * N * K / t / 1e12 / BF16_PEAK_TFLOPS,
                            "weight_gbs": w.size / t / 1e9}
        out[name] = {"N": N, "K": K, "by_m": by_m}
        W.free()
        dx.free()
        dy.free()
    return {"config": "prefill GEMM M sweeps (uq_gemm); q4k is the prefill workload N=12288 K=4096",
            "by_m": out["q4k"]["by_m"], "q6k": out["q6k"], "q80": out["q80"]}


def bench_gemm_q8k(hip, steps, warmup):
    """Bit-exact batched prefill (uq_gemm_q8k: every row gemv_quant_q8k, the
    reference forward's numerics) over M: Q4_K N=12288 K=4096 (the prefill
    workload) and Q6_K N=4096 K=12288; per_row_gemv_us is one uq_gemv_q8k
    call (M of them is what the reference's token-serial prefill issues)."""
    s = hip.stream()
    out = {}
    for dt, name, K, N in ((S.Q4_K, "q4k", 4096, 12288), (S.Q6_K, "q6k", 12288, 4096)):
        w = S.weights(dt, N, K, seed=S.seed_for(3))
        W = uq.Weights(w, dt, K, N)
        X = S.activations(K, seed=S.seed_for(3), rows=512)
        dx, dy = uq.DeviceArray.from_numpy(X), uq.DeviceArray(4 * 512 * N)
        by_m = {}
        for M in (1, 8, 32, 128, 512):
            st = max(10, steps // (1 if M < 128 else 2))
            wall, ev = timed(hip, lambda: uq.gemm_q8k(W, M, dx, dy, s), st, max(warmup, 20), s)
            t = ev * 1e-3 / st
            by_m[str(M)] = {"us": t * 1e6, "tflops": 2 * M * N * K / t / 1e12,
                            "frac_bf16_peak": 2 * M * N * K / t / 1e12 / BF16_PEAK_TFLOPS,
                            "weight_gbs": w.size / t / 1e9}
        out[name] = {"N": N, "K": K, "by_m": by_m, "per_row_gemv_us": by_m["1"]["us"]}
        W.free()
        dx.free()
        dy.free()
    return {"config": "bit-exact prefill GEMM (uq_gemm_q8k, gemv_quant_q8k per row) M sweeps; q4k is the prefill "
                      "workload N=12288 K=4096", **out}


def decode_layers():
    """Synthetic Qwen3.5-style hybrid 9B: 32 layers, hidden 4096; layer il is
    full attention when (il+1) % 4 == 0 (qwen35.rs:289-291), else GatedDeltaNet.
    Attention-block projections and ffn_down of the 8 attention layers are
    Q6_K, everything else Q4_K; Q6_K head with vocab 152064."""
    n, nff = 4096, 12288
    layers = []
    for il in range(32):
        attn = (il + 1) % 4 == 0
        dt = S.Q6_K if attn else S.Q4_K
        if attn:
            proj = [("attn_q", dt, n, 8192), ("attn_k", dt, n, 1024), ("attn_v", dt, n, 1024),
                    ("attn_output", dt, n, n)]
        else:
            proj = [("attn_qkv", S.Q4_K, n, 8192), ("attn_gate", S.Q4_K, n, n), ("ssm_beta", S.Q4_K, n, 32),
                    ("ssm_alpha", S.Q4_K, n, 32), ("ssm_out", S.Q4_K, n, n)]
        ffn = [("ffn_gate", S.Q4_K, n, nff), ("ffn_up", S.Q4_K, n, nff), ("ffn_down", dt, nff, n)]
        layers.append((attn, proj, ffn))
    return layers


class DecodeStep:
    """All quantized linear layers of one decode step of the synthetic hybrid
    9B, weights device-resident. Every layer reads the token's layer input x
    (N(0,1), f32); within a layer the projections chain as in the forward:
    the projections of x (batched), the output projection of the block (its
    input stands in for the GDN / attention result: the z gate output of a
    GDN layer, the first 4096 of q for attention), then gate/up with SwiGLU
    on that output and down on h. Each launch writes its own buffer, so one
    step leaves every launch's input and output in HBM for checking.
    Tensors of one shape share their host bytes (seeded once per shape)."""

    def __init__(self, head_h=None):
        n, nff = 4096, 12288
        self.n, self.nff = n, nff
        self.host = {}
        self.layers = []
        self.total = 0
        for attn, proj, ffn in decode_layers():
            L = {"attn": attn, "w": [], "shape": []}
            for name, dt, K, N in proj + ffn:
                L["w"].append(uq.Weights(self.bytes_of(dt, K, N), dt, K, N))
                L["shape"].append((name, dt, K, N))
                self.total += S.row_bytes(dt, K) * N
            sizes = ({"a": 8192, "c": 1024, "d": 1024} if attn else {"a": 8192, "b": n, "e": 32, "f": 32})
            sizes.update({"o": n, "g": nff, "u": nff, "h": nff, "y": n})
            L["buf"] = {k: uq.DeviceArray(4 * v) for k, v in sizes.items()}
            L["size"] = sizes
            self.layers.append(L)
        # the head's bytes are those of the head workload (seed of config 1)
        self.head_host = None if head_h is not None else S.weights(S.Q6_K, 152064, n, seed=S.seed_for(1))
        self.head = head_h if head_h is not None else uq.Weights(self.head_host, uq.DType.Q6K, n, 152064)
        self.total += S.row_bytes(S.Q6_K, n) * 152064
        self.x_host = S.activations(n, seed=S.seed_for(4))
        self.x = uq.DeviceArray.from_numpy(self.x_host)
        self.logits = uq.DeviceArray(4 * 152064)

    def bytes_of(self, dt, K, N):
        key = (dt, K, N)
        if key not in self.host:
            self.host[key] = S.weights(dt, N, K, seed=S.seed_for(4, len(self.host) + 1))
        return self.host[key]

    def chain(self, s, q8k=False):
        """Issue the step's launches on stream s (gemv_quant semantics, or
        the reference forward's gemv_quant_q8k for every projection)."""
        batch, one = (uq.gemv_q8k_batch, uq.gemv_q8k) if q8k else (uq.gemv_batch, uq.gemv)
        for L in self.layers:
            B, Wt = L["buf"], L["w"]
            if L["attn"]:
                q, k, v, o, g, u, d = Wt
                batch([q, k, v], self.x, [B["a"], B["c"], B["d"]], s)
                one(o, B["a"], B["o"], s)
            else:
                qkv, z, beta, alpha, o, g, u, d = Wt
                batch([qkv, z, beta, alpha], self.x, [B["a"], B["b"], B["e"], B["f"]], s)
                one(o, B["b"], B["o"], s)
            if q8k:
                uq.ffn_swiglu_q8k(g, u, d, B["o"], B["g"], B["u"], B["h"], B["y"], s)
            else:
                uq.ffn_swiglu(g, u, d, B["o"], B["h"], B["y"], s)
        one(self.head, self.x, self.logits, s)

    def launches(self):
        return sum(4 for _ in self.layers) + 1

    def free(self):
        for L in self.layers:
            for W in L["w"]:
                W.free()


def bench_decode(hip, steps, warmup, head_h=None):
    st = DecodeStep(head_h)
    s = hip.stream()
    graph = hip.capture(s, lambda: st.chain(s))
    wall, ev = timed(hip, lambda: hip.launch_graph(graph, s), steps, warmup, s)
    t = ev * 1e-3 / steps
    graph8 = hip.capture(s, lambda: st.chain(s, q8k=True))
    _, ev8 = timed(hip, lambda: hip.launch_graph(graph8, s), steps, warmup, s)
    t8 = ev8 * 1e-3 / steps
    total = st.total
    res = {"config": "decode step, synthetic hybrid 9B (32 layers, 24 GDN + 8 attention, FFN 12288, "
                     "Q6_K head 152064), all quantized linear layers in one HIP graph; projections of one input "
                     "batched (uq_gemv_batch); every layer reads the N(0,1) layer input",
           "weight_bytes_per_token": total, "launches": st.launches(), "ms_per_token": t * 1e3,
           "tok_s": 1.0 / t, "gbs": total / t / 1e9, "frac_hbm_peak": total / t / 1e9 / HBM_PEAK_GBS,
           "tok_s_wall": steps / wall,
           "q8k": {"semantics": "gemv_quant_q8k for every projection, the reference forward's numerics: every "
                                "projection bit-exact given its input; h = swiglu within 2 ulp (expf)",
                   "ms_per_token": t8 * 1e3, "tok_s": 1.0 / t8, "gbs": total / t8 / 1e9}}
    res["forward"] = bench_forward(hip, steps, warmup, st)
    st.free()
    return res


QWEN35_9B = dict(n_embd=4096, n_ff=12288, n_qk_heads=16, n_v_heads=32, head_dim_linear=128, conv_kernel=4,
                 n_head=16, n_head_kv=4, head_dim=256, n_rot=64)


def bench_forward(hip, steps, warmup, st, ctx=512):
    """The whole decode forward of one token on device: 24 GatedDeltaNet and
    8 attention layers (uq_gdn_layer_step_d / uq_attn_layer_step_d, the
    reference's recr_layer / attn_layer with gemv_quant_q8k projections),
    each layer's input the previous layer's output, then result_norm and the
    head; one HIP graph, attention at position ctx - 1 over a filled cache.
    Uses the decode step's weights; norms, conv kernels and gates are
    synthetic vectors shared by the layers of one kind."""
    from uq import layer as L
    from uq import ops as UO

    sh = QWEN35_9B
    theta = float(np.float32(1.0e7) ** np.float32(-2.0 / sh["n_rot"]))
    kq = float(np.float32(1.0) / np.sqrt(np.float32(sh["head_dim"])))
    d = L.Dims(**sh, theta_scale=theta, kq_scale=kq, rms_eps=1e-6)
    n, nv, hd, kv = sh["n_embd"], sh["n_v_heads"], sh["head_dim_linear"], sh["n_head_kv"] * sh["head_dim"]
    rng = np.random.default_rng(5)
    keep = []

    def dv(a):
        arr = uq.DeviceArray.from_numpy(np.ascontiguousarray(a, np.float32))
        keep.append(arr)
        return arr

    def norm(m):
        return dv(1.0 + 0.1 * rng.standard_normal(m))

    gvec = dict(attn_norm=norm(n), ssm_dt_bias=dv(rng.standard_normal(nv)),
                ssm_a=dv(-np.exp(0.5 * rng.standard_normal(nv))),
                ssm_conv1d=dv(0.3 * rng.standard_normal(d.channels * sh["conv_kernel"])), ssm_norm=norm(hd),
                post_attention_norm=norm(n))
    avec = dict(attn_norm=norm(n), attn_q_norm=norm(sh["head_dim"]), attn_k_norm=norm(sh["head_dim"]),
                post_attention_norm=norm(n))
    layers = []
    for Lr in st.layers:
        Wt = Lr["w"]
        if Lr["attn"]:
            q, k, v, o, g, u, dn = Wt
            w = L.AttnWeights(attn_q=q, attn_k=k, attn_v=v, attn_output=o, ffn_gate=g, ffn_up=u, ffn_down=dn, **avec)
            layers.append(("attn", w, dv(rng.standard_normal(ctx * kv) / 16), dv(rng.standard_normal(ctx * kv))))
        else:
            qkv, z, beta, alpha, o, g, u, dn = Wt
            w = L.GdnWeights(attn_qkv=qkv, attn_gate=z, ssm_beta=beta, ssm_alpha=alpha, ssm_out=o, ffn_gate=g,
                             ffn_up=u, ffn_down=dn, **gvec)
            layers.append(("gdn", w, dv(np.zeros(sh["conv_kernel"] * d.channels)), dv(np.zeros(nv * hd * hd))))
    ws = uq.DeviceArray(4 * L.ws_floats(d, ctx))
    xa, xb, xn = uq.DeviceArray(4 * n), uq.DeviceArray(4 * n), uq.DeviceArray(4 * n)
    out_norm = norm(n)
    s = hip.stream()

    def chain():
        x = st.x
        for i, (kind, w, a, b) in enumerate(layers):
            y = xa if i % 2 == 0 else xb
            if kind == "gdn":
                L.gdn_step(d, w, a, b, x, y, ws, s)
            else:
                L.attn_step(d, w, a, b, ctx, ctx - 1, x, y, ws, s)
            x = y
        UO.rmsnorm_d(xn, x, out_norm, n, 1, 1e-6, s)  # result_norm (min_forward.rs:187-205)
        uq.gemv_q8k(st.head, xn, st.logits, s)        # output_logits (min_forward.rs:207-266)

    graph = hip.capture(s, chain)
    wall, ev = timed(hip, lambda: hip.launch_graph(graph, s), steps, warmup, s)
    t = ev * 1e-3 / steps

    # prefill: P tokens through the same 32 layers, one prefill call per layer
    # (projections and FFNs as q8k GEMMs over the P tokens, bit-identical to P
    # steps); launched eagerly from the host. P = 128 and P = ctx (512).
    def prefill_run(P):
        xp = uq.DeviceArray.from_numpy(rng.standard_normal(P * n).astype(np.float32))
        pa, pb = uq.DeviceArray(4 * P * n), uq.DeviceArray(4 * P * n)
        pws = uq.DeviceArray(4 * max(L.prefill_ws_floats(d, P, gdn=w, n_ctx_max=0) if kind == "gdn" else
                                     L.prefill_ws_floats(d, P, attn=w, n_ctx_max=ctx) for kind, w, _, _ in layers))

        def prefill():
            x = xp
            for i, (kind, w, a, b) in enumerate(layers):
                y = pa if i % 2 == 0 else pb
                if kind == "gdn":
                    L.gdn_prefill(d, w, a, b, P, x, y, pws, s)
                else:
                    L.attn_prefill(d, w, a, b, ctx, 0, P, x, y, pws, s)
                x = y

        _, evp = timed(hip, prefill, 3, 1, s)
        tp = evp * 1e-3 / 3
        for a in (xp, pa, pb, pws):
            a.free()
        return {"config": f"{P} tokens at positions 0..{P - 1} through the 32 layers (no head), one "
                          f"uq_gdn_layer_prefill_d / uq_attn_layer_prefill_d call per layer, launched "
                          f"eagerly; every output equals {P} one-token steps bit for bit",
                "tokens": P, "ms": tp * 1e3, "tok_s": P / tp, "token_serial_ms_estimate": P * t * 1e3,
                "speedup_vs_token_serial": P * t / tp}

    pre = prefill_run(128)
    pre512 = prefill_run(ctx)
    for a in keep + [ws, xa, xb, xn]:
        a.free()
    return {"config": f"one decode token through the device-resident forward: 24 GatedDeltaNet + 8 attention "
                      f"layers of the synthetic hybrid 9B with their FFNs, result_norm and the Q6_K head, "
                      f"gemv_quant_q8k projections, attention at position {ctx - 1}; one HIP graph",
            "ms_per_token": t * 1e3, "tok_s": 1.0 / t, "weight_bytes_per_token": st.total,
            "gbs": st.total / t / 1e9, "prefill": pre, f"prefill_{ctx}": pre512}


def cpu_baseline(w, x):
    """The oracle (C restatement of quants.rs's scalar kernels) on the first
    third of the head, 1 thread, median of 3; plus all cores."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    K, rows = 4096, 152064 // 3
    ws = w[: rows * S.row_bytes(S.Q6_K, K)]
    out = np.zeros(rows, np.float32)
    nbytes = gemv_bytes(S.Q6_K, K, rows)

    def rate(fn, nt, reps):
        ts = []
        for _ in range(reps):
            t = time.perf_counter()
            fn(out, x, ws, K, rows, S.Q6_K, nthreads=nt)
            ts.append(time.perf_counter() - t)
        return nbytes / statistics.median(ts) / 1e9

    ncpu = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    ncpu = min(ncpu, 16)
    q8k_1 = rate(O.gemv_quant_q8k, 1, 3)
    exact_1 = rate(O.gemv_quant, 1, 3)
    q8k_all = rate(O.gemv_quant_q8k, ncpu, 3)
    return {"value": q8k_1, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"gemv_quant_q8k (the reference forward's path) over rows 0..{rows} of the same "
                      f"Q6_K head, C restatement of quants.rs built -O2 -ffp-contract=off, median of 3",
            "gemv_quant_exact_1core_gbs": exact_1, "q8k_all_cores_gbs": q8k_all, "all_cores": ncpu,
            **host_cpu(), "nproc": os.cpu_count()}


def host_cpu():
    """The host CPU as /proc/cpuinfo reports it: the full model string of the
    first processor, its family / model / stepping numbers, clock, cache and
    vector extensions, and the count of logical processors listed."""
    first, n = {}, 0
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("processor"):
                    n += 1
                if n == 1 and ":" in line:
                    k, v = line.split(":", 1)
                    first.setdefault(k.strip(), v.strip())
    except OSError:
        pass
    flags = set(first.get("flags", "").split())
    return {"cpu_model": first.get("model name", "unknown"),
            "cpu_vendor": first.get("vendor_id"), "cpu_family": first.get("cpu family"),
            "cpu_model_number": first.get("model"), "cpu_stepping": first.get("stepping"),
            "cpu_mhz": first.get("cpu MHz"), "cpu_cache": first.get("cache size"),
            "cpu_vector_ext": sorted(flags & {"avx2", "avx512f", "avx512bw", "avx512_vnni", "avx512_bf16", "fma"}),
            "cpuinfo_processors": n}


def load_traffic():
    """HBM bytes per launch of the head GEMV from the committed counter
    summary (FETCH_SIZE + WRITE_SIZE, each scaled by the same counter's
    reading for a device-to-device copy of known size)."""
    p = os.path.join(PROFILES, "q6k_head_gemv_counters.md")
    try:
        with open(p) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except (OSError, ValueError):
        pass
    return None


def copy_calibration(nbytes=1 << 30):
    """One device-to-device copy of a known size, so a counter run
    (FETCH_SIZE / WRITE_SIZE) has a reference dispatch to scale by."""
    a, b = uq.DeviceArray(nbytes), uq.DeviceArray(nbytes)
    for _ in range(2):
        uq.lib().uq_memcpy_dtod(b.ptr, a.ptr, nbytes, None)
    uq.synchronize()
    log(f"copy calibration: 2 device-to-device copies of {nbytes} bytes")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="headline workload only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="", help="comma list of: head,q4k,q4k_large,ffn,gemm,gemm_q8k,decode")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run two 1 GiB device copies (reference dispatches for counter runs)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {a.gpus} is not supported (the path runs on a single "
              f"MI355X; the row-sharded design is documented with the sources).", file=sys.stderr)
        sys.exit(2)
    hip = Hip()
    log("device:", uq.device_name())
    if a.copy_calibration:
        copy_calibration()
    only = set(filter(None, a.only.split(",")))
    head, w, x, W = bench_head(hip, a.steps, a.warmup)
    extra = {"head_q8k_bit_exact": head["q8k"]}
    if not a.quick:
        for name, fn in (("q4k", bench_q4k_small), ("q4k_large", bench_q4k_large), ("ffn", bench_ffn),
                         ("gemm", bench_gemm), ("gemm_q8k", bench_gemm_q8k)):
            if not only or name in only:
                log("bench:", name)
                extra[name] = fn(hip, a.steps, a.warmup)
        if not only or "decode" in only:
            log("bench: decode")
            extra["decode"] = bench_decode(hip, max(5, a.steps // 2), 2, head_h=W)
    cpu = None if a.no_cpu else cpu_baseline(w, x)
    ach = head["gbs_event"]
    line = {
        "metric": METRIC, "value": head["gbs_wall"], "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": head["wall_s"] * 1e3 / a.steps, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "i8-dot4/f64",
        "data": "synthetic (seeded random GGUF blocks, N(0,1) activations)",
        "config": {"workload": "Q6_K output-projection GEMV 152064x4096 (gemv_quant semantics)",
                   "dim_out": 152064, "dim_in": 4096, "weight_bytes": 510935040,
                   "algorithmic_bytes_per_step": head["bytes"]},
        "roofline": {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": ach / HBM_PEAK_GBS, "traffic": load_traffic()},
        "cpu_baseline": cpu,
        "extra": extra,
        "host": platform.node(),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
