"""GPU parity of the resident decode chain (aspida_kq_chain_*).

Every step of a chain is checked against the oracle's QMatVec on the input the
step actually read (the chain's own earlier outputs), within MV_RTOL times
sum_i |w_i x_i| per output -- over every kind, ragged row counts, column
counts that leave waves idle (3, 7 super-blocks), inputs at an offset inside
a producer's output, independent steps that share an input, and the
Llama-3-8B decoder shapes.  Runs are deterministic, reusable (each launch is
a new epoch of the ready flags), replay from a HIP graph, and report no
abandoned dependency wait.
"""
import numpy as np
import pytest

import aspida_amd as aa
import oracle
from aspida_amd import synth
from gpu_helpers import abs_dot_scale, assert_close_scaled, ncpu, stream, sync, to_dev, torch_cuda

pytestmark = pytest.mark.gpu


class Arena:
    """One device f32 buffer holding every activation vector, 64-float aligned."""

    def __init__(self, sizes):
        torch = torch_cuda()
        self.off, n = {}, 0
        for name, size in sizes:
            self.off[name] = (n, size)
            n += (size + 63) // 64 * 64
        self.buf = torch.zeros(n, dtype=torch.float32, device="cuda")

    def ptr(self, name, start=0):
        return self.buf.data_ptr() + 4 * (self.off[name][0] + start)

    def get(self, name, start=0, count=None):
        o, size = self.off[name]
        count = size - start if count is None else count
        return self.buf[o + start:o + start + count].cpu().numpy()

    def put(self, name, arr):
        torch = torch_cuda()
        o, size = self.off[name]
        assert arr.size == size
        self.buf[o:o + size] = torch.from_numpy(arr).cuda()


def _build(dev, spec, gen):
    """spec: [(name, kind, out, in, (src, start) or None for an input)]; returns
    arena, weights, packed tensors and the chain."""
    torch = torch_cuda()
    sizes = [("x0", max(s[3] for s in spec if s[4] is None))] + [(s[0], s[2]) for s in spec]
    ar = Arena(sizes)
    W, keep, steps = {}, [], []
    for name, kind, out, inp, src in spec:
        w = synth.weight_np(kind, out, inp, gen)
        raw = to_dev(w)
        p = torch.empty(dev.packed_bytes(kind, inp, out), dtype=torch.uint8, device="cuda")
        dev.pack(kind, raw.data_ptr(), inp, out, p.data_ptr(), stream())
        W[name] = w
        keep += [raw, p]
        xs, start = ("x0", 0) if src is None else src
        steps.append((kind, p.data_ptr(), inp, out, ar.ptr(xs, start), ar.ptr(name)))
    sync()
    return ar, W, keep, dev.chain(steps)


def _check(ar, W, spec, what):
    for name, kind, out, inp, src in spec:
        xs, start = ("x0", 0) if src is None else src
        x = ar.get(xs, start, inp)
        y = ar.get(name)
        want = oracle.qmatvec(kind, W[name], inp, out, x, nthreads=ncpu())
        assert_close_scaled(y, want, abs_dot_scale(kind, W[name], inp, out, x), what=f"{what} step {name}")


MIXED = [
    # name, kind, out, in, x source (step, start) -- None: the launch input x0
    ("a", aa.Q4_K, 1536, 1024, None),
    ("b", aa.Q6_K, 512, 1024, None),             # shares x0 with a, no dependency
    ("c", aa.Q5_K, 1024, 1536, ("a", 0)),
    ("d", aa.Q3_K, 2048, 512, ("a", 512)),       # x at an offset inside a's output
    ("e", aa.Q2_K, 300, 2048, ("d", 0)),         # ragged rows
    ("f", aa.Q8_0, 256, 1792, ("d", 256)),       # 7 columns: one unit with an idle wave
    ("g", aa.Q4_K, 4096, 768, ("a", 768)),       # 3 columns: five idle waves per unit
    ("h", aa.Q6_K, 640, 1024, ("c", 0)),
]


def test_chain_mixed_kinds_and_offsets():
    dev = aa.DeviceOps()
    gen = synth.rng(4242)
    ar, W, keep, ch = _build(dev, MIXED, gen)
    try:
        for rep in range(3):                     # a new epoch per launch
            ar.put("x0", synth.activations_np(1024, gen))
            ch.run(stream())
            sync()
            assert ch.check(), "a dependency wait gave up"
            _check(ar, W, MIXED, f"run {rep}")
    finally:
        ch.close()


def test_chain_deterministic_and_graph_replay():
    torch = torch_cuda()
    dev = aa.DeviceOps()
    gen = synth.rng(777)
    ar, W, keep, ch = _build(dev, MIXED, gen)
    try:
        ar.put("x0", synth.activations_np(1024, gen))
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            ch.run(s.cuda_stream)
            s.synchronize()
            first = ar.buf.cpu().numpy().copy()
            ch.run(s.cuda_stream)
            s.synchronize()
            assert np.array_equal(first.view(np.uint32), ar.buf.cpu().numpy().view(np.uint32))
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                ch.run(s.cuda_stream)
            for _ in range(3):
                ar.buf.zero_()
                ar.put("x0", first[:1024].copy())
                g.replay()
                s.synchronize()
                assert np.array_equal(first.view(np.uint32), ar.buf.cpu().numpy().view(np.uint32)), "graph replay"
        assert ch.check()
    finally:
        ch.close()


def _decoder_spec(layers):
    H, F, KV = 4096, 14336, 1024
    spec = []
    prev = None
    for l in range(layers):
        spec += [(f"qk{l}", aa.Q4_K, H + KV, H, prev),
                 (f"v{l}", aa.Q6_K, KV, H, prev),
                 (f"o{l}", aa.Q4_K, H, H, (f"qk{l}", 0)),
                 (f"gu{l}", aa.Q4_K, 2 * F, H, (f"o{l}", 0)),
                 (f"dn{l}", aa.Q6_K, H, F, (f"gu{l}", 0))]
        prev = (f"dn{l}", 0)
    return spec


def test_chain_decoder_layers():
    """Two Llama-3-8B layers (q|k, v, o, gate|up, down), each input the
    previous output, run three times in a row."""
    dev = aa.DeviceOps()
    gen = synth.rng(31337)
    spec = _decoder_spec(2)
    ar, W, keep, ch = _build(dev, spec, gen)
    try:
        for rep in range(3):                     # a new epoch per launch
            ar.put("x0", synth.activations_np(4096, gen))
            ch.run(stream())
            sync()
            assert ch.check()
            _check(ar, W, spec, f"decoder run {rep}")
        assert ch.workgroups() >= 16 and ch.workgroups() % 16 == 0
    finally:
        ch.close()
