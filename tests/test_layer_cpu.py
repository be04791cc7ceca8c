"""The layer API's host-side checks (include/uq_layer.h) without a GPU: the
workspace layout and the refusals that come before any launch."""
import ctypes as C

import pytest

import uq
from uq import layer as L

SMALL = dict(n_embd=512, n_ff=1024, n_qk_heads=4, n_v_heads=8, head_dim_linear=64, conv_kernel=4, n_head=4,
             n_head_kv=2, head_dim=128, n_rot=32)


def dims(**over):
    s = dict(SMALL, **over)
    return L.Dims(**s, theta_scale=0.5, kq_scale=0.088, rms_eps=1e-6)


def test_workspace_layout():
    d = dims()
    prev_end = 0
    for name in L.NODES:
        off, cnt = L.node_at(d, name, 16)
        assert off % 64 == 0 and off >= prev_end, name
        prev_end = off + cnt
    assert L.ws_floats(d, 16) >= prev_end
    # only the softmax rows depend on n_ctx_max, and they come last
    for name in L.NODES[:-1]:
        assert L.node_at(d, name, 0) == L.node_at(d, name, 1000), name
    assert L.node_at(d, "soft", 16)[1] == 4 * 16
    assert L.node_at(d, "conv_silu")[1] == 2 * 4 * 64 + 8 * 64


@pytest.mark.parametrize("over", [dict(n_embd=0), dict(conv_kernel=1), dict(conv_kernel=10), dict(n_v_heads=6),
                                  dict(head_dim=96), dict(n_head_kv=3), dict(n_rot=33), dict(n_rot=256)])
def test_bad_dims_are_refused(over):
    d = dims(**over)
    assert L.ws_floats(d) == 0
    with pytest.raises(uq.UqError) as e:
        L.node_at(d, "z")
    assert e.value.kind == "ARG"


def test_step_refuses_bad_handles_before_launching():
    d = dims()

    class Null:
        ptr = None
        h = None
        nbytes = 4 * L.ws_floats(d, 8)

    gw = L.GdnWeights(*([Null()] * 14))
    with pytest.raises(uq.UqError) as e:
        L.gdn_step(d, gw, Null(), Null(), Null(), Null(), Null())
    assert e.value.kind == "ARG" and "null pointer" in str(e.value)
    aw = L.AttnWeights(*([Null()] * 11))
    with pytest.raises(uq.UqError) as e:
        L.attn_step(d, aw, Null(), Null(), 8, 0, Null(), Null(), Null())
    assert e.value.kind == "ARG"
