"""GPU: one mask classification per graph (mxfa_graph_begin / mxfa_graph_end).

The reference builds each mask once per graph and hands the same tensor to
every layer's attention node (src/qwen3-lm.h:515-517 -> :541-543;
src/dit-graph.h:522-528 -> :574-576).  Inside a begin/end bracket the engine
classifies such a mask at its first node only.  These tests check that
  * the nodes of one graph launch the classifier once per distinct mask, and
    produce outputs bit-identical to calls that classify per call;
  * a new graph after the mask's contents changed reclassifies them;
  * the same data pointer under another shape (Sq) is a different mask;
  * a captured graph reclassifies at every replay, following contents the
    host rewrites in place between replays.
"""
from __future__ import annotations

import contextlib
import gc

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
D = 128


@pytest.fixture(scope="module")
def mx():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import mxfa

    return mxfa


@contextlib.contextmanager
def no_gc():
    gc.collect()
    gc.disable()
    try:
        yield
    finally:
        gc.enable()


class Problem:
    """Prefill-shaped FA inputs: Q F32 [D, Sq, Nh, 1], K/V F16 [D, Skv, Nkv, 1],
    an F16 mask [Skv, Sq, 1, 1] and its own output per query set."""

    def __init__(self, mx, Sq=512, Skv=512, Nh=8, Nkv=2, n_q=3, seed=0):
        import torch

        g = torch.Generator(device="cpu").manual_seed(seed)
        self.mx, self.Sq, self.Skv, self.Nh, self.Nkv = mx, Sq, Skv, Nh, Nkv
        self.qs = [torch.randn(Nh, Sq, D, generator=g).cuda() for _ in range(n_q)]
        self.k = torch.randn(Nkv, Skv, D, generator=g).half().cuda()
        self.v = torch.randn(Nkv, Skv, D, generator=g).half().cuda()
        self.mask = torch.zeros(Sq, Skv, dtype=torch.float16, device="cuda")
        self.outs = [torch.zeros(Sq, Nh, D, device="cuda") for _ in range(n_q)]

    def set_causal(self, shift):
        """Key j live for query i iff j <= i + shift (a causal mask with an
        offset, which moves the diagonal across tile boundaries)."""
        import torch

        i = torch.arange(self.Sq, device="cuda")[:, None]
        j = torch.arange(self.Skv, device="cuda")[None, :]
        self.mask.copy_(torch.where(j <= i + shift, 0.0, float("-inf")).half())

    def set_padding(self, live):
        import torch

        j = torch.arange(self.Skv, device="cuda")[None, :].expand(self.Sq, -1)
        self.mask.copy_(torch.where(j < live, 0.0, float("-inf")).half())

    def views(self, i, sq=None, mask=None, out=None):
        mx, Nh, Nkv, Skv = self.mx, self.Nh, self.Nkv, self.Skv
        sq = self.Sq if sq is None else sq
        m = self.mask if mask is None else mask
        o = self.outs[i] if out is None else out
        q = self.qs[i]
        qv = mx.DeviceView(0, (D, sq, Nh, 1), (4, 4 * D, 4 * D * self.Sq, 4 * D * self.Sq * Nh), q.data_ptr(), q)
        kv = mx.DeviceView(1, (D, Skv, Nkv, 1), (2, 2 * D, 2 * D * Skv, 2 * D * Skv * Nkv), self.k.data_ptr(),
                           self.k)
        vv = mx.DeviceView(1, (D, Skv, Nkv, 1), (2, 2 * D, 2 * D * Skv, 2 * D * Skv * Nkv), self.v.data_ptr(),
                           self.v)
        mv = mx.DeviceView(1, (Skv, sq, 1, 1), (2, 2 * Skv, 2 * Skv * self.Sq, 2 * Skv * self.Sq), m.data_ptr(), m)
        ov = mx.DeviceView(0, (D, Nh, sq, 1), (4, 4 * D, 4 * D * Nh, 4 * D * Nh * sq), o.data_ptr(), o)
        return qv, kv, vv, mv, ov

    def call(self, i, stream=None, **kw):
        qv, kv, vv, mv, ov = self.views(i, **kw)
        self.mx.flash_attn_ext(qv, kv, vv, mv, D ** -0.5, dst=ov, stream=stream)


def per_call(p, i, **kw):
    """Reference output: the same call outside any graph (classified per call)."""
    import torch

    out = torch.zeros_like(p.outs[i])
    p.call(i, out=out, **kw)
    torch.cuda.synchronize()
    return out.clone()


def classifier_launches(mx, fn):
    import torch

    torch.cuda.synchronize()
    mx.timing_reset()
    mx.timing_enable(True)
    try:
        fn()
        torch.cuda.synchronize()
    finally:
        mx.timing_enable(False)
    _, n_cls = mx.timing_read("mask_classify")
    _, n_fa = mx.timing_read("fa_prefill")
    mx.timing_reset()
    return n_cls, n_fa


def test_one_classification_per_graph(mx):
    import torch

    p = Problem(mx, seed=1)
    p.set_causal(0)
    refs = [per_call(p, i) for i in range(3)]

    def graph():
        with mx.graph():
            for i in range(3):
                p.call(i)

    n_cls, n_fa = classifier_launches(mx, graph)
    assert (n_cls, n_fa) == (1, 3)
    for i in range(3):
        assert torch.equal(p.outs[i], refs[i]), i
    # outside the bracket every call classifies again
    n_cls, n_fa = classifier_launches(mx, lambda: [p.call(i) for i in range(3)])
    assert (n_cls, n_fa) == (3, 3)


def test_new_contents_new_graph_reclassify(mx):
    import torch

    p = Problem(mx, seed=2)
    for shift in (0, 37, -100):
        p.set_causal(shift)
        refs = [per_call(p, i) for i in range(2)]
        with mx.graph():
            p.call(0)
            p.call(1)
        torch.cuda.synchronize()
        for i in range(2):
            assert torch.equal(p.outs[i], refs[i]), (shift, i)
    # a padding mask in the same buffer: tiles that were mixed become all
    # zero or all -inf
    p.set_padding(200)
    refs = [per_call(p, i) for i in range(2)]
    n_cls, _ = classifier_launches(mx, lambda: (mx.graph_begin(), p.call(0), p.call(1), mx.graph_end()))
    assert n_cls == 1
    for i in range(2):
        assert torch.equal(p.outs[i], refs[i]), i


def test_two_masks_and_two_shapes_in_one_graph(mx):
    import torch

    p = Problem(mx, seed=3)
    p.set_causal(5)
    m2 = torch.where(torch.arange(p.Skv, device="cuda")[None, :].expand(p.Sq, -1) < 300, 0.0,
                     float("-inf")).half().contiguous()
    ref_a = per_call(p, 0)
    ref_b = per_call(p, 1, mask=m2)
    ref_c = per_call(p, 2, sq=256)   # the first 256 rows of the same mask buffer
    outs = [torch.zeros_like(o) for o in p.outs]

    def graph():
        with mx.graph():
            p.call(0, out=outs[0])
            p.call(1, mask=m2, out=outs[1])
            p.call(2, sq=256, out=outs[2])
            p.call(0, out=outs[0])
            p.call(1, mask=m2, out=outs[1])

    n_cls, n_fa = classifier_launches(mx, graph)
    assert (n_cls, n_fa) == (3, 5)
    assert torch.equal(outs[0], ref_a)
    assert torch.equal(outs[1], ref_b)
    assert torch.equal(outs[2][:256], ref_c[:256])


def test_captured_graph_reclassifies_every_replay(mx):
    import torch

    p = Problem(mx, seed=4)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    p.set_causal(0)
    torch.cuda.synchronize()
    # eager run of the graph on the capture stream: sizes its workspace and
    # its class arena
    with torch.cuda.stream(s):
        with mx.graph(s.cuda_stream):
            p.call(0, stream=s.cuda_stream)
            p.call(1, stream=s.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    mx.graph_begin(s.cuda_stream)
    try:
        with no_gc():
            with torch.cuda.stream(s):
                with torch.cuda.graph(g, stream=s):
                    p.call(0, stream=s.cuda_stream)
                    p.call(1, stream=s.cuda_stream)
    finally:
        mx.graph_end(s.cuda_stream)
    torch.cuda.synchronize()
    for shift in (0, 64, -64, 200, 0):
        p.set_causal(shift)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in p.outs[:2]]
        # eager work between replays, outside any graph bracket
        refs = [per_call(p, i) for i in range(2)]
        for i in range(2):
            assert torch.equal(got[i], refs[i]), (shift, i)
        assert np.isfinite(got[0].cpu().numpy()).all()
