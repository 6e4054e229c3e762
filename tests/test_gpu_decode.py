"""Whole-model decode on the GPU against the oracle (bit-exact with the
reference's forward(), test_oracle.py): per-layer hidden states within 1e-3
relative L2 (observed ~1e-6), identical greedy tokens,
eager and HIP-graph loops identical, and the host-hidden drop-in for
cuda_transformer_layer_gpu keeping the host KV cache coherent."""
import numpy as np
import pytest

from guanaco_amd import spec as S
from util import rel_l2

pytestmark = pytest.mark.gpu

LAYER_TOL = 1e-3


@pytest.fixture(scope="module")
def tiny(ctx, orc):
    import guanaco_amd.hip as H
    spec, ms, pre = S.TINY_TEST, 64, 24
    from oracle import HostModel
    hm = HostModel(orc, spec, ms)
    dm = H.DeviceModel(ctx, spec, ms, prefill=pre)
    return spec, ms, pre, hm, dm


@pytest.mark.parametrize("path", ["auto", "valu", "mfma"])
def test_forward_per_layer_and_tokens(ctx, orc, tiny, path):
    import guanaco_amd.hip as H
    spec, ms, pre, hm, dm = tiny
    with H.matvec_path(path):
        _forward_per_layer_and_tokens(ctx, orc, spec, pre, hm, dm)


def _forward_per_layer_and_tokens(ctx, orc, spec, pre, hm, dm):
    ctx.kv_prefill_synth(*[__import__("guanaco_amd.synth").synth.tensor_seed(spec.seed, -1, s)
                           for s in (13, 14)], pre)
    kv = hm.new_kv()
    kv.prefill(orc, spec, pre)
    tok = 11
    worst = 0.0
    for step in range(6):
        t_gpu, lg, hg = dm.forward(tok, pre + step, want_hidden=True)
        t_cpu, lc, hc = hm.forward(kv, tok, pre + step, want_hidden=True)
        for l in range(spec.n_layers):
            e = rel_l2(hg[l], hc[l])
            worst = max(worst, e)
            assert e < LAYER_TOL, (step, l, e)
        assert rel_l2(lg, lc) < LAYER_TOL
        assert t_gpu == t_cpu, step
        tok = t_cpu
    print("worst per-layer rel L2", worst)


@pytest.mark.parametrize("name", ["tiny-test", "wide-ff-test"])
def test_q6k_unit_layout_bit_identical(name):
    """The Q6_K down projection read from the vector-ALU unit layout (the
    copy gq_hip_model_bind makes; 4-row groups in the 1024-thread launches
    of wide-ff's 28672-column rows) gives the reference layout's results bit
    for bit: the same products in the same order."""
    import guanaco_amd.hip as H
    from util import bits
    spec = S.PRESETS[name]
    c = H.Context(0)
    try:
        ms, pre = 64, 24
        dm = H.DeviceModel(c, spec, ms, prefill=pre)
        out = {}
        for path in ("auto", "auto_q6k_ref"):
            with H.matvec_path(path):
                c.kv_prefill_synth(11, 12, pre)
                out[path] = [dm.forward(7 + i, pre + i, want_hidden=True) for i in range(3)]
        for a, b in zip(out["auto"], out["auto_q6k_ref"]):
            assert a[0] == b[0]
            assert np.array_equal(bits(a[1]), bits(b[1])) and np.array_equal(bits(a[2]), bits(b[2]))
    finally:
        c.close()


def test_forward_q6k_down_odd_blocks(orc):
    """A Q6_K down projection whose rows hold an odd count of 256-column
    blocks (ff 768) gets no unit-layout copy (its rows would start at a
    2-byte phase) and reads the reference layout: per-layer hidden states and
    tokens against the oracle as for the other models."""
    import guanaco_amd.hip as H
    from oracle import HostModel
    spec = S.ModelSpec("odd-ff-test", n_layers=2, hidden=512, ff=768, n_heads=8, n_kv_heads=2, vocab=1000,
                       layer_dtypes=dict(wd=S.Q6_K))
    c = H.Context(0)
    try:
        ms, pre = 64, 24
        hm = HostModel(orc, spec, ms)
        dm = H.DeviceModel(c, spec, ms, prefill=pre)
        _forward_per_layer_and_tokens(c, orc, spec, pre, hm, dm)
    finally:
        c.close()


def test_graph_loop_matches_eager_and_oracle(ctx, orc, tiny):
    spec, ms, pre, hm, dm = tiny
    from guanaco_amd.synth import tensor_seed
    seeds = (tensor_seed(spec.seed, -1, 13), tensor_seed(spec.seed, -1, 14))
    n = 24
    ctx.kv_prefill_synth(*seeds, pre)
    eager, _ = dm.decode_loop(5, pre, n, use_graph=False)
    ctx.kv_prefill_synth(*seeds, pre)
    graph, _ = dm.decode_loop(5, pre, n, use_graph=True)
    ctx.kv_prefill_synth(*seeds, pre)
    graph2, _ = dm.decode_loop(5, pre, n, use_graph=True)  # replays of the same graph
    kv = hm.new_kv()
    kv.prefill(orc, spec, pre)
    tok, cpu = 5, []
    for i in range(n):
        tok, _, _ = hm.forward(kv, tok, pre + i)
        cpu.append(tok)
    assert list(eager) == cpu
    assert list(graph) == cpu and list(graph2) == cpu


def test_decode_rejects_positions_past_cache(ctx, tiny):
    import guanaco_amd.hip as H
    spec, ms, pre, hm, dm = tiny
    with pytest.raises(H.HipError):
        dm.decode_loop(1, ms - 2, 4)
    with pytest.raises(H.HipError):
        dm.forward(1, ms)


def test_transformer_layer_host_mirror(ctx, orc, tiny):
    """gq_hip_transformer_layer: host hidden in/out for one layer, new K/V
    rows written back into the host cache (fixes the stale host cache of the
    CUDA path)."""
    spec, ms, pre, hm, dm = tiny
    from guanaco_amd.synth import tensor_seed
    ctx.kv_prefill_synth(tensor_seed(spec.seed, -1, 13), tensor_seed(spec.seed, -1, 14), pre)
    kv = hm.new_kv()
    kv.prefill(orc, spec, pre)
    h0 = orc.synth_normal(3, spec.hidden)
    import ctypes as C
    from oracle import fptr
    hc = h0.copy()
    orc.lib.orc_layer(C.byref(hm.s), C.byref(kv.s), 0, pre, fptr(hc))
    n = spec.n_kv_heads * ms * spec.head_dim
    hk = np.zeros(n, np.float32)
    hv = np.zeros(n, np.float32)
    rc, hg = dm.transformer_layer(0, pre, h0, hk, hv, ms * spec.head_dim)
    assert rc == 0 and rel_l2(hg, hc) < LAYER_TOL
    dk, dv = ctx.kv_read_layer(0)
    for h in range(spec.n_kv_heads):
        sl = slice((h * ms + pre) * spec.head_dim, (h * ms + pre + 1) * spec.head_dim)
        assert np.array_equal(hk[sl], dk[sl]) and np.array_equal(hv[sl], dv[sl])
        assert rel_l2(dk[sl], kv.k[sl]) < LAYER_TOL


def test_fused_qkv_rope_append_bitexact(ctx, orc, tiny):
    """The decode path's fused q/k/v epilogue (RoPE + K/V append inside the
    matvec) equals plain matvecs followed by the standalone RoPE+append kernel
    (itself bit-exact against the reference's rope + kv_cache_append)."""
    import guanaco_amd.hip as H
    from util import bits
    spec, ms, pre, hm, dm = tiny
    hd, nkv = spec.head_dim, spec.n_kv_heads
    h = ctx.upload(orc.synth_normal(8, spec.hidden) * np.float32(3))
    q1, q2 = ctx.alloc(4 * spec.hidden), ctx.alloc(4 * spec.hidden)
    pos, layer = pre + 3, 1
    assert H.lib.gq_hip_qkv_rope_dev(ctx.h, layer, pos, h.ptr, q1.ptr, 0) == 0
    k1, v1 = ctx.kv_read_layer(layer)
    z = np.zeros_like(k1)
    ctx.kv_write_layer(layer, z, z)
    assert H.lib.gq_hip_qkv_rope_dev(ctx.h, layer, pos, h.ptr, q2.ptr, 1) == 0
    k2, v2 = ctx.kv_read_layer(layer)
    assert np.array_equal(bits(q1.download()), bits(q2.download()))
    r1 = lambda a: a.reshape(nkv, ms, hd)[:, pos]  # noqa: E731
    assert np.abs(r1(k2)).sum() > 0 and np.abs(r1(v2)).sum() > 0
    assert np.array_equal(bits(r1(k1)), bits(r1(k2))) and np.array_equal(bits(r1(v1)), bits(r1(v2)))
    # nothing else in the slab was written
    k2r = k2.reshape(nkv, ms, hd).copy()
    k2r[:, pos] = 0
    assert not k2r.any()


def test_profile_step_accounts_every_launch(ctx, tiny):
    spec, ms, pre, hm, dm = tiny
    prof = dm.profile_step(3, pre)
    # per layer: qkv (one launch per distinct dtype), o, gate/up, down; LM head
    assert spec.n_layers <= prof["qkv"]["launches"] <= 3 * spec.n_layers
    for k in ("attention", "o_proj", "gate_up", "down"):
        assert prof[k]["launches"] == spec.n_layers, k
    assert prof["lm_head"]["launches"] == 1 and prof["other"]["launches"] == 2
    assert all(v["ms"] >= 0 for v in prof.values())
