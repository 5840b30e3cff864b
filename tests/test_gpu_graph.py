"""GPU: HIP graph capture and replay of a decode step (the reference's static
decode graph: src/static-graph.h, src/qwen3-lm.h:36-58, and the per-layer
KV write + attention of :448-469).

A step of L layers -- KV-cache write of K and V (mxfa_set_rows), then
attention over the cache window (mxfa_flash_attn_ext with the causal mask) --
is captured once into a graph (torch.cuda.graph over the engine's stream)
and replayed for several tokens.  Between replays the host rewrites the
static inputs in place (new rows, row id, mask, queries), as the reference
does, and runs eager work on the device.  Every replay's outputs and caches
must equal, bit for bit, an eager twin that runs the same calls on its own
copy of the state.
"""
from __future__ import annotations

import contextlib
import gc

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
D = 128


@contextlib.contextmanager
def no_gc():
    """No garbage collection while a stream is being captured: a collected
    cycle that owns device tensors or graphs would release them in the
    middle of the capture, which the runtime refuses (abort)."""
    gc.collect()
    gc.disable()
    try:
        yield
    finally:
        gc.enable()


@pytest.fixture(scope="module")
def mx():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import mxfa

    return mxfa


class Step:
    """Static buffers of one decode step (fixed addresses, as in a graph)."""

    def __init__(self, mx, L, Nh, Nkv, max_seq, n_kv_pad, seed):
        import torch

        g = torch.Generator(device="cpu").manual_seed(seed)
        self.mx, self.L, self.Nh, self.Nkv, self.max_seq, self.n_kv_pad = mx, L, Nh, Nkv, max_seq, n_kv_pad
        dev = "cuda"
        self.cache_k = [(torch.randn(Nkv, max_seq, D, generator=g) * 0.5).half().to(dev) for _ in range(L)]
        self.cache_v = [(torch.randn(Nkv, max_seq, D, generator=g) * 0.5).half().to(dev) for _ in range(L)]
        self.k_new = [torch.zeros(Nkv, 1, D, device=dev) for _ in range(L)]
        self.v_new = [torch.zeros(Nkv, 1, D, device=dev) for _ in range(L)]
        self.q = [torch.zeros(Nh, 1, D, device=dev) for _ in range(L)]
        self.rows = torch.zeros(1, dtype=torch.int64, device=dev)
        self.mask = torch.zeros(1, n_kv_pad, dtype=torch.float16, device=dev)
        self.out = [torch.zeros(1, 1, Nh, D, device=dev) for _ in range(L)]

    def views(self, l):
        mx, Nh, Nkv, ms, W = self.mx, self.Nh, self.Nkv, self.max_seq, self.n_kv_pad
        kc, vc = self.cache_k[l], self.cache_v[l]
        cache_nb = (2, 2 * D, 2 * D * ms, 2 * D * ms * Nkv)
        dk = mx.DeviceView(1, (D, ms, Nkv, 1), cache_nb, kc.data_ptr(), kc)
        dv = mx.DeviceView(1, (D, ms, Nkv, 1), cache_nb, vc.data_ptr(), vc)
        kwin = mx.DeviceView(1, (D, W, Nkv, 1), cache_nb, kc.data_ptr(), kc)
        vwin = mx.DeviceView(1, (D, W, Nkv, 1), cache_nb, vc.data_ptr(), vc)
        src_nb = (4, 4 * D, 4 * D, 4 * D * Nkv)
        ks = mx.DeviceView(0, (D, 1, Nkv, 1), src_nb, self.k_new[l].data_ptr(), self.k_new[l])
        vs = mx.DeviceView(0, (D, 1, Nkv, 1), src_nb, self.v_new[l].data_ptr(), self.v_new[l])
        rows = mx.DeviceView(27, (1, 1, 1, 1), (8, 8, 8, 8), self.rows.data_ptr(), self.rows)
        q = mx.DeviceView(0, (D, 1, Nh, 1), (4, 4 * D, 4 * D, 4 * D * Nh), self.q[l].data_ptr(), self.q[l])
        m = mx.DeviceView(1, (W, 1, 1, 1), (2, 2 * W, 2 * W, 2 * W), self.mask.data_ptr(), self.mask)
        o = mx.DeviceView(0, (D, Nh, 1, 1), (4, 4 * D, 4 * D * Nh, 4 * D * Nh), self.out[l].data_ptr(),
                          self.out[l])
        return dk, dv, kwin, vwin, ks, vs, rows, q, m, o

    def run(self, stream=None):
        """The step's launches, in the reference's order."""
        for l in range(self.L):
            dk, dv, kwin, vwin, ks, vs, rows, q, m, o = self.views(l)
            self.mx.set_rows(dk, ks, rows, stream=stream)
            self.mx.set_rows(dv, vs, rows, stream=stream)
            self.mx.flash_attn_ext(q, kwin, vwin, m, 1.0 / D ** 0.5, dst=o, stream=stream)

    def set_inputs(self, pos, seed):
        """Host-side input update of one token (in place, fixed addresses)."""
        import torch

        g = torch.Generator(device="cpu").manual_seed(seed)
        for l in range(self.L):
            self.k_new[l].copy_(torch.randn(self.Nkv, 1, D, generator=g))
            self.v_new[l].copy_(torch.randn(self.Nkv, 1, D, generator=g))
            self.q[l].copy_(torch.randn(self.Nh, 1, D, generator=g))
        self.rows.fill_(pos)
        j = torch.arange(self.n_kv_pad)
        self.mask.copy_(torch.where(j <= pos, 0.0, float("-inf")).half().view(1, -1))


def test_decode_step_graph_replays_match_eager(mx):
    import torch

    L, Nh, Nkv, max_seq, W = 4, 16, 8, 1024, 512
    graph_state = Step(mx, L, Nh, Nkv, max_seq, W, seed=1)
    eager_state = Step(mx, L, Nh, Nkv, max_seq, W, seed=1)
    base = 300
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    # eager warm-up of the graph's own buffers on the capture stream sizes
    # that stream's workspace (the engine keeps one per stream)
    graph_state.set_inputs(base - 1, seed=99)
    with torch.cuda.stream(s):
        graph_state.run(stream=s.cuda_stream)
    eager_state.set_inputs(base - 1, seed=99)
    eager_state.run()
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    with no_gc(), torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            graph_state.run(stream=s.cuda_stream)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    for step in range(4):
        pos = base + step
        print(f"[graph] replay {step} at position {pos}", flush=True)
        graph_state.set_inputs(pos, seed=step)
        eager_state.set_inputs(pos, seed=step)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        eager_state.run()                    # eager work between replays
        _ = torch.randn(1 << 20, device="cuda").sum()
        torch.cuda.synchronize()
        for l in range(L):
            assert torch.equal(graph_state.out[l], eager_state.out[l]), (step, l)
            assert torch.equal(graph_state.cache_k[l], eager_state.cache_k[l]), (step, l)
            assert torch.equal(graph_state.cache_v[l], eager_state.cache_v[l]), (step, l)
        # the new token's rows were written, and attention saw them
        assert float(graph_state.out[0].abs().sum()) > 0


def test_growth_under_capture_is_refused(mx):
    """A call whose workspace would have to grow while the stream is being
    captured fails cleanly (no allocation, nothing launched); after
    mxfa_reserve the same call captures and replays."""
    import torch

    from mxfa import cases as C

    c = C.lm_batch("t", N=8, Nh=32, Nkv=8, max_seq=8192, lmin=6000, lmax=8192)   # a large split workspace
    mx.release()
    dq, dk, dv, dm = mx.upload(c.q), mx.upload(c.k), mx.upload(c.v), mx.upload(c.mask)
    B, Sq, Nh, DV = c.out_shape
    out = torch.zeros(B, Sq, Nh, DV, device="cuda")
    dst = mx.DeviceView(0, (DV, Nh, Sq, B), (4, 4 * DV, 4 * DV * Nh, 4 * DV * Nh * Sq), out.data_ptr(), out)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    status, detail = None, ""
    with no_gc(), torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            try:
                mx.flash_attn_ext(dq, dk, dv, dm, c.scale, dst=dst, stream=s.cuda_stream)
            except mx.MxfaError as e:
                # keep the status only: the exception's traceback would tie
                # this frame (graphs, tensors) into a cycle
                status, detail = e.status, e.detail
    torch.cuda.synchronize()
    assert status == mx.ERR_UNSUPPORTED, (status, detail)
    assert "captured" in detail
    mx.reserve(dq, dk, dv, dm, c.scale, stream=s.cuda_stream)
    g2 = torch.cuda.CUDAGraph()
    with no_gc(), torch.cuda.stream(s):
        with torch.cuda.graph(g2, stream=s):
            mx.flash_attn_ext(dq, dk, dv, dm, c.scale, dst=dst, stream=s.cuda_stream)
    torch.cuda.synchronize()
    ref = torch.zeros_like(out)
    refv = mx.DeviceView(0, dst.ne, dst.nb, ref.data_ptr(), ref)
    for _ in range(3):
        out.zero_()
        g2.replay()
        torch.cuda.synchronize()
        mx.flash_attn_ext(dq, dk, dv, dm, c.scale, dst=refv)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)

    # A larger eager call on the capture stream grows its workspace after
    # the capture: the outgrown buffers the graph holds are retired, not
    # freed, so the graph still replays correctly (interleaved with the
    # grown workspace's own calls).
    _, retired0 = mx.workspace_info()
    # 16 query rows per KV head need 4x the partials of the one-token batch
    big = C.lm_single("t2", n_tokens=16, kv_pos=7000, Nh=32, Nkv=8, max_seq=8192)
    bq, bk, bv, bm = mx.upload(big.q), mx.upload(big.k), mx.upload(big.v), mx.upload(big.mask)
    Bb, Sqb, Nhb, DVb = big.out_shape
    bout = torch.zeros(Bb, Sqb, Nhb, DVb, device="cuda")
    bdst = mx.DeviceView(0, (DVb, Nhb, Sqb, Bb), (4, 4 * DVb, 4 * DVb * Nhb, 4 * DVb * Nhb * Sqb), bout.data_ptr(), bout)
    with torch.cuda.stream(s):
        mx.flash_attn_ext(bq, bk, bv, bm, big.scale, dst=bdst, stream=s.cuda_stream)
    torch.cuda.synchronize()
    live, retired1 = mx.workspace_info()
    assert retired1 > retired0, (retired0, retired1, live)
    for _ in range(2):
        out.zero_()
        with torch.cuda.stream(s):
            g2.replay()
            mx.flash_attn_ext(bq, bk, bv, bm, big.scale, dst=bdst, stream=s.cuda_stream)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
    del g, g2
    torch.cuda.synchronize()
    gc.collect()


class FusedStep:
    """A decode step with the pre-attention fusion: per layer one
    mxfa_qk_norm_rope (QK-norm, RoPE, 16-bit cast, K/V written into their
    cache row) and one attention call on the F16 Q it wrote -- the layer's
    two launches in place of the reference's op chain
    (src/qwen3-lm.h:418-469)."""

    def __init__(self, mx, L, Nh, Nkv, max_seq, n_kv_pad, seed):
        import torch

        g = torch.Generator(device="cpu").manual_seed(seed)
        self.mx, self.L, self.Nh, self.Nkv, self.max_seq, self.W = mx, L, Nh, Nkv, max_seq, n_kv_pad
        dev = "cuda"
        H = Nh + 2 * Nkv
        self.x = [torch.zeros(1, 1, H, D, device=dev) for _ in range(L)]
        self.w = [(1 + 0.2 * torch.randn(2, D, generator=g)).to(dev) for _ in range(L)]
        self.cache_k = [(torch.randn(Nkv, max_seq, D, generator=g) * 0.5).half().to(dev) for _ in range(L)]
        self.cache_v = [(torch.randn(Nkv, max_seq, D, generator=g) * 0.5).half().to(dev) for _ in range(L)]
        self.q16 = [torch.zeros(1, 1, Nh, D, dtype=torch.float16, device=dev) for _ in range(L)]
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.rows = torch.zeros(1, dtype=torch.int64, device=dev)
        self.mask = torch.zeros(1, n_kv_pad, dtype=torch.float16, device=dev)
        self.out = [torch.zeros(1, 1, Nh, D, device=dev) for _ in range(L)]

    def run(self, stream=None):
        mx, Nh, Nkv, ms, W = self.mx, self.Nh, self.Nkv, self.max_seq, self.W
        H = Nh + 2 * Nkv
        V = mx.DeviceView
        for l in range(self.L):
            x, w, kc, vc, q16, o = self.x[l], self.w[l], self.cache_k[l], self.cache_v[l], self.q16[l], self.out[l]
            xnb = (4, 4 * D, 4 * D * H, 4 * D * H)
            cnb = (2, 2 * D, 2 * D * ms, 2 * D * ms * Nkv)
            wnb = (4, 4 * D, 4 * D, 4 * D)
            mx.qk_norm_rope(V(0, (D, Nh, 1, 1), xnb, x.data_ptr(), x),
                            V(0, (D, Nkv, 1, 1), xnb, x.data_ptr() + 4 * D * Nh, x),
                            V(0, (D, Nkv, 1, 1), xnb, x.data_ptr() + 4 * D * (Nh + Nkv), x),
                            V(0, (D, 1, 1, 1), wnb, w.data_ptr(), w), V(0, (D, 1, 1, 1), wnb, w.data_ptr() + 4 * D, w),
                            V(26, (1, 1, 1, 1), (4, 4, 4, 4), self.pos.data_ptr(), self.pos), 1e-6, 1e6,
                            V(1, (D, Nh, 1, 1), (2, 2 * D, 2 * D * Nh, 2 * D * Nh), q16.data_ptr(), q16),
                            V(1, (D, ms, Nkv, 1), cnb, kc.data_ptr(), kc), V(1, (D, ms, Nkv, 1), cnb, vc.data_ptr(), vc),
                            V(27, (1, 1, 1, 1), (8, 8, 8, 8), self.rows.data_ptr(), self.rows), stream=stream)
            mx.flash_attn_ext(V(1, (D, 1, Nh, 1), (2, 2 * D * Nh, 2 * D, 2 * D * Nh), q16.data_ptr(), q16),
                              V(1, (D, W, Nkv, 1), cnb, kc.data_ptr(), kc), V(1, (D, W, Nkv, 1), cnb, vc.data_ptr(), vc),
                              V(1, (W, 1, 1, 1), (2, 2 * W, 2 * W, 2 * W), self.mask.data_ptr(), self.mask),
                              1.0 / D ** 0.5,
                              dst=V(0, (D, Nh, 1, 1), (4, 4 * D, 4 * D * Nh, 4 * D * Nh), o.data_ptr(), o),
                              stream=stream)

    def set_inputs(self, pos, seed):
        import torch

        g = torch.Generator(device="cpu").manual_seed(seed)
        for l in range(self.L):
            self.x[l].copy_(torch.randn(self.x[l].shape, generator=g) * 2)
        self.pos.fill_(pos)
        self.rows.fill_(pos)
        j = torch.arange(self.W)
        self.mask.copy_(torch.where(j <= pos, 0.0, float("-inf")).half().view(1, -1))


def test_fused_decode_step_graph_replays_match_eager(mx):
    """The fused decode layer (pre-attention step + attention on its F16 Q)
    captured for 4 layers and replayed for 4 tokens, each replay equal bit
    for bit to an eager twin, caches included."""
    import torch

    L, Nh, Nkv, max_seq, W = 4, 16, 8, 1024, 512
    gs = FusedStep(mx, L, Nh, Nkv, max_seq, W, seed=3)
    es = FusedStep(mx, L, Nh, Nkv, max_seq, W, seed=3)
    base = 200
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    gs.set_inputs(base - 1, seed=77)
    with torch.cuda.stream(s):
        gs.run(stream=s.cuda_stream)     # sizes the capture stream's workspace
    es.set_inputs(base - 1, seed=77)
    es.run()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with no_gc(), torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            gs.run(stream=s.cuda_stream)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for step in range(4):
        pos = base + step
        print(f"[graph fused] replay {step} at position {pos}", flush=True)
        gs.set_inputs(pos, seed=10 + step)
        es.set_inputs(pos, seed=10 + step)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        es.run()
        _ = torch.randn(1 << 20, device="cuda").sum()
        torch.cuda.synchronize()
        for l in range(L):
            assert torch.equal(gs.out[l], es.out[l]), (step, l)
            assert torch.equal(gs.q16[l], es.q16[l]), (step, l)
            assert torch.equal(gs.cache_k[l], es.cache_k[l]), (step, l)
            assert torch.equal(gs.cache_v[l], es.cache_v[l]), (step, l)
        assert float(gs.out[0].abs().sum()) > 0
        # the token's cache row holds the step's K (not the warm-up's)
        assert not torch.equal(gs.cache_k[0][:, pos], torch.zeros_like(gs.cache_k[0][:, pos]))


def test_device_lengths_follow_graph_replays(mx):
    """Structured masks with device-resident lengths (MXFA_MASK_DEVICE): a
    C3-shaped batched decode (8 sequences, 32/8 heads, cache 8192) captured
    once and replayed for 4 tokens while the host rewrites the per-sequence
    lengths (and the query) between replays, as the reference's static
    decode graph does with its kv_len inputs (src/qwen3-lm.h:864-884).  Each
    replay equals an eager call with the same device lengths bit for bit,
    and the dense-mask call at the parity bar; no mask tensor exists."""
    import torch

    from conftest import MAX_ABS_TOL, ROW_COS_TOL, row_metrics
    from mxfa import cases as C

    c = C.c3()
    N, Nh, Dh = 8, 32, 128
    dk, dv = mx.upload(c.k), mx.upload(c.v)
    g = torch.Generator(device="cpu").manual_seed(5)
    q = torch.zeros(N, Nh, 1, Dh, device="cuda")
    qv = mx.DeviceView(0, (Dh, 1, Nh, N), (4, 4 * Dh, 4 * Dh, 4 * Dh * Nh), q.data_ptr(), q)
    lens = torch.tensor(c.meta["lengths"], dtype=torch.int32, device="cuda")
    spec = mx.mask_spec(device_lengths=lens)
    out = torch.zeros(N, 1, Nh, Dh, device="cuda")
    ov = mx.DeviceView(0, (Dh, Nh, 1, N), (4, 4 * Dh, 4 * Dh * Nh, 4 * Dh * Nh), out.data_ptr(), out)
    ref = torch.zeros_like(out)
    rv = mx.DeviceView(0, ov.ne, ov.nb, ref.data_ptr(), ref)
    dense = torch.zeros_like(out)
    dvw = mx.DeviceView(0, ov.ne, ov.nb, dense.data_ptr(), dense)
    n_kv = int(c.k.ne[1])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        mx.flash_attn_ext_masked(qv, dk, dv, spec, c.scale, dst=ov, stream=s.cuda_stream)   # sizes s's workspace
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with no_gc(), torch.cuda.stream(s):
        with torch.cuda.graph(gr, stream=s):
            mx.flash_attn_ext_masked(qv, dk, dv, spec, c.scale, dst=ov, stream=s.cuda_stream)
    torch.cuda.synchronize()
    base = [int(x) for x in c.meta["lengths"]]
    for step in range(4):
        new = [min(n_kv, L - 300 * step + 7 * step * (i % 3)) for i, L in enumerate(base)]
        print(f"[graph device lengths] replay {step}: {new}", flush=True)
        q.copy_(torch.randn(q.shape, generator=g))
        lens.copy_(torch.tensor(new, dtype=torch.int32))
        torch.cuda.synchronize()
        out.zero_()
        gr.replay()
        torch.cuda.synchronize()
        mx.flash_attn_ext_masked(qv, dk, dv, spec, c.scale, dst=rv)
        j = torch.arange(n_kv, device="cuda")
        mask = torch.where(j[None, :] < torch.tensor(new, device="cuda")[:, None], 0.0, float("-inf")).half()
        mview = mx.DeviceView(1, (n_kv, 1, 1, N), (2, 2 * n_kv, 2 * n_kv, 2 * n_kv), mask.data_ptr(), mask)
        mx.flash_attn_ext(qv, dk, dv, mview, c.scale, dst=dvw)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), step
        m = row_metrics(out.cpu().numpy(), dense.cpu().numpy())
        assert m["max_abs"] <= MAX_ABS_TOL and m["min_cos"] >= ROW_COS_TOL, (step, m)
    del gr
    torch.cuda.synchronize()
    gc.collect()


def test_device_pos0_prefill_equals_host_pos0(mx):
    """A causal prompt continuation with pos0 in device memory equals the
    same call with pos0 given on the host, bit for bit (prefill kernel)."""
    import torch

    from mxfa import cases as C

    c = C.lm_single("dp", n_tokens=300, kv_pos=211, Nh=16, Nkv=8, max_seq=1024)
    dq, dk, dv = mx.upload(c.q), mx.upload(c.k), mx.upload(c.v)
    p0 = torch.tensor([211], dtype=torch.int32, device="cuda")
    a = mx.flash_attn_ext_masked(dq, dk, dv, mx.mask_spec(causal=True, pos0=211), c.scale)
    b = mx.flash_attn_ext_masked(dq, dk, dv, mx.mask_spec(causal=True, device_pos0=p0), c.scale)
    torch.cuda.synchronize()
    assert torch.equal(mx.output_tensor(a), mx.output_tensor(b))


def test_device_lengths_and_pos0_wide_prefill(mx):
    """Structured calls of at most 4 key tiles run the kernel with 48 queries
    per wave; with lengths and pos0 in device memory they equal the same
    calls with host values, bit for bit, and follow new device values."""
    import torch

    from test_gpu_parity import _rand_case

    c = _rand_case(560, B=3, Sq=300, Nh=8, Nkv=2, Skv=200, mask=None)
    dq, dk, dv = mx.upload(c.q), mx.upload(c.k), mx.upload(c.v)
    lens = torch.tensor([200, 150, 37], dtype=torch.int32, device="cuda")
    p0 = torch.tensor([20], dtype=torch.int32, device="cuda")
    for host_lens, host_p0 in (([200, 150, 37], 20), ([90, 200, 0], 5)):
        lens.copy_(torch.tensor(host_lens, dtype=torch.int32))
        p0.fill_(host_p0)
        print(f"[wide device spec] lengths {host_lens} pos0 {host_p0}", flush=True)
        a = mx.flash_attn_ext_masked(dq, dk, dv, mx.mask_spec(causal=True, window=70, pos0=host_p0,
                                                                 lengths=host_lens), c.scale)
        b = mx.flash_attn_ext_masked(dq, dk, dv, mx.mask_spec(causal=True, window=70, device_pos0=p0,
                                                                 device_lengths=lens), c.scale)
        torch.cuda.synchronize()
        assert torch.equal(mx.output_tensor(a), mx.output_tensor(b))
