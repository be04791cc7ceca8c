"""GPU tests of the prefill layer forms (include/uq_layer.h): n tokens through
a GatedDeltaNet or full-attention layer in one call must give exactly what n
successive step calls give, bit for bit: every token's layer output, the
conv window and recurrent state after the last token, and the KV cache rows.

The reference prefills token by token (greedy.rs:55-65), so the step
(itself checked node by node against the oracle's recr_layer / attn_layer in
tests/test_gpu_layers.py) is the reference here. The prefill runs every
projection once over all tokens as uq_gemm_q8k and the norms, swiglu and
residual adds over all rows, and the GatedDeltaNet's recurrent part in one
launch over the tokens (head dims 64 and 128) or the step's launches per
token (other head dims); the counts cover the q8k GEMM's tile shapes
(1 token: the decode kernel; 5 and 16: 16-row tiles; 17-128: 32-row tiles;
130: 64-row tiles), windows and states carried from earlier tokens, conv
kernels of 2, 3, 4 and 9 taps, the attention starting at a position past
earlier tokens, the small model and the 9B shapes of the decode benchmark.
"""
import sys

import numpy as np
import pytest

import uq
from uq import layer as L
from test_gpu_layers import FULL, SMALL, Model, assert_bitwise

pytestmark = pytest.mark.gpu


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def tokens(n_embd, nt, seed):
    return np.random.default_rng(seed).standard_normal((nt, n_embd)).astype(np.float32)


def gdn_by_steps(m, X, win0, state0):
    c, d = m.cfg, m.d
    nt, n = X.shape
    win, state = uq.DeviceArray.from_numpy(win0), uq.DeviceArray.from_numpy(state0)
    ws = uq.DeviceArray(4 * L.ws_floats(d))
    dl = uq.DeviceArray(4 * n)
    out = np.empty_like(X)
    for t in range(nt):
        dx = uq.DeviceArray.from_numpy(X[t])
        L.gdn_step(d, m.gw, win, state, dx, dl, ws)
        out[t] = dl.download(np.float32, n)
        dx.free()
    res = out, win.download(np.float32, win.nbytes // 4), state.download(np.float32, state.nbytes // 4)
    for a in (win, state, ws, dl):
        a.free()
    return res


def gdn_by_prefill(m, X, win0, state0):
    c, d = m.cfg, m.d
    nt, n = X.shape
    win, state = uq.DeviceArray.from_numpy(win0), uq.DeviceArray.from_numpy(state0)
    ws = uq.DeviceArray(4 * L.prefill_ws_floats(d, nt, gdn=m.gw))
    dx, dl = uq.DeviceArray.from_numpy(X), uq.DeviceArray(4 * nt * n)
    L.gdn_prefill(d, m.gw, win, state, nt, dx, dl, ws)
    res = (dl.download(np.float32, nt * n).reshape(nt, n), win.download(np.float32, win.nbytes // 4),
           state.download(np.float32, state.nbytes // 4))
    for a in (win, state, ws, dx, dl):
        a.free()
    return res


def check_gdn(m, nt, seed, what, carried=False):
    """nt tokens from an empty window and state, or (carried) from a random
    window and state as earlier tokens leave them"""
    c = m.cfg
    X = tokens(c.n_embd, nt, seed)
    rng = np.random.default_rng(seed + 100)
    nwin, nstate = c.conv_kernel * m.d.channels, c.n_v_heads * c.head_dim_linear ** 2
    win0 = rng.standard_normal(nwin).astype(np.float32) if carried else np.zeros(nwin, np.float32)
    state0 = (0.05 * rng.standard_normal(nstate)).astype(np.float32) if carried else np.zeros(nstate, np.float32)
    ref_out, ref_win, ref_state = gdn_by_steps(m, X, win0, state0)
    out, win, state = gdn_by_prefill(m, X, win0, state0)
    for t in range(nt):
        assert_bitwise(out[t], ref_out[t], f"{what} token {t} l_out")
    assert_bitwise(win, ref_win, f"{what} conv window")
    assert_bitwise(state, ref_state, f"{what} state")
    assert np.all(np.isfinite(out))
    log(f"{what}: {nt} tokens bit-identical to {nt} steps")


# other GatedDeltaNet shapes: head_dim_linear 32 (the per-token launches)
# and 64 with the shortest and longest conv kernels (the one-launch scan;
# with 9 taps a short prefill keeps rows of the earlier window)
OTHER = dict(n_embd=256, n_ff=512, n_qk_heads=4, n_v_heads=8, head_dim_linear=32, conv_kernel=3, n_head=2,
             n_head_kv=1, head_dim=128, n_rot=32)


@pytest.mark.parametrize("hd,ck", [(32, 3), (64, 2), (64, 9)])
@pytest.mark.parametrize("nt", [1, 3, 11, 40])
def test_gdn_prefill_other_shapes_equal_steps(hd, ck, nt):
    shape = dict(OTHER, head_dim_linear=hd, conv_kernel=ck, n_embd=8 * hd, n_head=8 * hd // 128)
    m = Model(shape, seed=49 + hd + ck)
    check_gdn(m, nt, seed=nt + 3, what=f"gdn hd={hd} ck={ck}", carried=True)
    m.free()


def attn_run(m, X, n_ctx_max, pos0, prefill, warm):
    """warm tokens by steps (positions 0 .. pos0 - 1), then X at pos0 .. by
    steps or by one prefill call; returns X's outputs and both caches."""
    c, d = m.cfg, m.d
    nt, n = X.shape
    kv = c.n_head_kv * c.head_dim
    kc = uq.DeviceArray.from_numpy(np.zeros(n_ctx_max * kv, np.float32))
    vc = uq.DeviceArray.from_numpy(np.zeros(n_ctx_max * kv, np.float32))
    ws = uq.DeviceArray(4 * max(L.ws_floats(d, n_ctx_max), L.prefill_ws_floats(d, nt, attn=m.aw, n_ctx_max=n_ctx_max)))
    dl = uq.DeviceArray(4 * n)
    for p in range(pos0):
        dx = uq.DeviceArray.from_numpy(warm[p])
        L.attn_step(d, m.aw, kc, vc, n_ctx_max, p, dx, dl, ws)
        dx.free()
    if prefill:
        dx, dlm = uq.DeviceArray.from_numpy(X), uq.DeviceArray(4 * nt * n)
        L.attn_prefill(d, m.aw, kc, vc, n_ctx_max, pos0, nt, dx, dlm, ws)
        out = dlm.download(np.float32, nt * n).reshape(nt, n)
        dx.free()
        dlm.free()
    else:
        out = np.empty_like(X)
        for t in range(nt):
            dx = uq.DeviceArray.from_numpy(X[t])
            L.attn_step(d, m.aw, kc, vc, n_ctx_max, pos0 + t, dx, dl, ws)
            out[t] = dl.download(np.float32, n)
            dx.free()
    res = out, kc.download(np.float32, kc.nbytes // 4), vc.download(np.float32, vc.nbytes // 4)
    for a in (kc, vc, ws, dl):
        a.free()
    return res


def check_attn(m, nt, pos0, n_ctx_max, seed, what):
    X = tokens(m.cfg.n_embd, nt, seed)
    warm = tokens(m.cfg.n_embd, max(pos0, 1), seed + 1)
    ref = attn_run(m, X, n_ctx_max, pos0, False, warm)
    got = attn_run(m, X, n_ctx_max, pos0, True, warm)
    for t in range(nt):
        assert_bitwise(got[0][t], ref[0][t], f"{what} token {t} l_out")
    assert_bitwise(got[1], ref[1], f"{what} k cache")
    assert_bitwise(got[2], ref[2], f"{what} v cache")
    assert np.all(np.isfinite(got[0]))
    log(f"{what}: {nt} tokens from position {pos0} bit-identical to {nt} steps")


@pytest.mark.parametrize("q6", [False, True])
@pytest.mark.parametrize("nt", [1, 5, 16, 17, 40, 130])
def test_gdn_prefill_small_equals_steps(nt, q6):
    m = Model(SMALL, seed=41 + q6)
    check_gdn(m, nt, seed=nt, what=f"gdn small q6={q6}", carried=nt in (5, 40))
    m.free()


@pytest.mark.parametrize("q6", [False, True])
@pytest.mark.parametrize("nt,pos0", [(1, 0), (5, 3), (16, 0), (40, 7), (130, 2)])
def test_attn_prefill_small_equals_steps(nt, pos0, q6):
    m = Model(SMALL, seed=43 + q6)
    check_attn(m, nt, pos0, n_ctx_max=256, seed=nt + pos0, what=f"attn small q6={q6}")
    m.free()


@pytest.mark.parametrize("head_dim,n_head,n_head_kv", [(64, 8, 2), (512, 1, 1)])
def test_attn_prefill_head_dims_equal_steps(head_dim, n_head, n_head_kv):
    """Attention heads of 64 (the one-lane-per-position scores kernel at its
    smallest tree) and of 512 (beyond it: the step's scores kernel over the
    token dimension)."""
    m = Model(dict(SMALL, n_head=n_head, n_head_kv=n_head_kv, head_dim=head_dim, n_rot=32), seed=53 + head_dim)
    check_attn(m, 70, 4, n_ctx_max=128, seed=head_dim, what=f"attn head_dim={head_dim}")
    m.free()


@pytest.mark.parametrize("shape,nt", [
    (dict(n_embd=768, n_v_heads=12, n_head=6, n_head_kv=2, head_dim=128), 37),
    (dict(n_head=8, n_head_kv=1, head_dim=64), 19),
    (dict(n_embd=1280, n_v_heads=20, n_head=5, n_head_kv=1, head_dim=256), 23)])
def test_attn_prefill_head_groups_equal_steps(shape, nt):
    """Head groups of 3, 8 and 5 q heads per kv head: the prefill's pv
    kernel takes 16 / group queries per workgroup (5, 2 and 3 here), the
    last block of each run partly filled."""
    m = Model(dict(SMALL, **shape), seed=61 + shape["n_head"])
    check_attn(m, nt, 5, n_ctx_max=96, seed=shape["n_head"], what=f"attn {shape}")
    m.free()


def test_attn_prefill_chunked_equals_steps():
    """A context so long that the scores of 40 tokens exceed the prefill's
    2^24-float scores area: the attention runs in chunks of 15, 15 and 10
    tokens (n_head 4 x n_ctx_max 262145 floats per token)."""
    m = Model(SMALL, seed=51)
    check_attn(m, 40, 3, n_ctx_max=262145, seed=11, what="attn small chunked")
    m.free()


def test_prefill_9b_shapes_equal_steps():
    """The decode benchmark's 9B shapes: 20 tokens through a GatedDeltaNet
    layer and 12 through an attention layer after 5 earlier positions."""
    m = Model(FULL, seed=45)
    check_gdn(m, 20, seed=7, what="gdn 9b")
    check_gdn(m, 9, seed=9, what="gdn 9b carried", carried=True)
    check_attn(m, 12, 5, n_ctx_max=64, seed=8, what="attn 9b")
    m.free()


def test_prefill_refusals_and_empty_call():
    m = Model(SMALL, seed=47)
    d, c = m.d, m.cfg
    kv = c.n_head_kv * c.head_dim
    kc, vc = uq.DeviceArray(4 * 8 * kv), uq.DeviceArray(4 * 8 * kv)
    X = tokens(c.n_embd, 4, 1)
    dx, dl = uq.DeviceArray.from_numpy(X), uq.DeviceArray(4 * X.size)
    ws = uq.DeviceArray(4 * L.prefill_ws_floats(d, 4, attn=m.aw, n_ctx_max=8))
    with pytest.raises(uq.UqError) as e:  # positions 5..8 with n_ctx_max 8: context full
        L.attn_prefill(d, m.aw, kc, vc, 8, 5, 4, dx, dl, ws)
    assert e.value.kind == "ARG"
    small = uq.DeviceArray(4 * 64)
    with pytest.raises(uq.UqError) as e:  # workspace too small
        L.attn_prefill(d, m.aw, kc, vc, 8, 0, 4, dx, dl, small)
    assert e.value.kind == "ARG"
    L.attn_prefill(d, m.aw, kc, vc, 8, 0, 0, dx, dl, small)  # no tokens: nothing to do
    assert L.prefill_ws_floats(d, 0, attn=m.aw) == 0
    for a in (kc, vc, dx, dl, ws, small):
        a.free()
    m.free()
