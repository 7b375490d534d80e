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


# ---- resident model chain (the reference's chain ABI: aspida_gpu_chain_*) -------------
#
# A small MoE model registered through aspida_kq_chain_layer + aspida_gpu_chain_moe +
# aspida_gpu_chain_model, checked against oracle.chain_forward (LLM_Qwen_Blk.Step with a
# matvec mixer, LLM_MoE.Forward, final norm and head): the residual stream after every
# layer, then the logits, for single tokens, lane batches and graph replays.  The bound is
# CHAIN_RTOL of the largest |value| of the compared vector: every step is an f32 sum in
# another order than the CPU's (norms, matvecs, router, experts), compounded over layers.
CHAIN_RTOL = 2e-4

Q4, Q5, Q6, Q8 = aa.Q4_K, aa.Q5_K, aa.Q6_K, aa.Q8_0

# mixer kind (None: no mixer, -1: f32), router kind (-1: f32), expert kinds (gate, up,
# down, shared gate, shared up, shared down), gated shared expert
SMALL_LAYERS = [
    (Q4, -1, (Q4, Q4, Q6, Q4, Q4, Q6), True),    # grouped, matrix-core kinds
    (Q6, Q8, (Q5, Q5, Q8, Q5, Q5, Q8), True),    # grouped, vector-ALU kinds; quantised router
    (None, -1, (Q4, Q5, Q6, Q4, Q4, Q6), False),  # mixed gate/up kinds: per-projection kernels
    (-1, Q4, (Q4, Q4, Q6, Q4, Q4, Q6), True),    # dense f32 mixer
]


def _mat(kind, out, inp, gen, scale=0.05):
    if kind == -1:
        return (gen.normal(0.0, scale, (out, inp)).astype(np.float32), -1)
    return (synth.weight_np(kind, out, inp, gen), kind)


def _chain_model(gen, dim, inter, n_exp, top_k, vocab, rows, layers):
    norm = lambda: (1.0 + 0.1 * gen.standard_normal(dim)).astype(np.float32)
    M = {"embed": gen.standard_normal((rows, dim)).astype(np.float32), "fnorm": norm(),
         "lm": _mat(Q6, vocab, dim, gen), "vocab": vocab, "layers": []}
    for mix, rk, kinds, gated in layers:
        gk, uk, dk, sgk, suk, sdk = kinds
        M["layers"].append({
            "attn_norm": norm(), "post_norm": norm(),
            "mix": None if mix is None else _mat(mix, dim, dim, gen, 0.02),
            "moe": {"router": _mat(rk, n_exp, dim, gen, 0.1),
                    "gate": _mat(gk, n_exp * inter, dim, gen), "up": _mat(uk, n_exp * inter, dim, gen),
                    "down": _mat(dk, n_exp * dim, inter, gen), "shg": _mat(sgk, inter, dim, gen),
                    "shu": _mat(suk, inter, dim, gen), "shd": _mat(sdk, dim, inter, gen),
                    "sgi": gen.normal(0.0, 0.05, dim).astype(np.float32) if gated else None,
                    "n_exp": n_exp, "top_k": top_k, "intermed": inter}})
    return M


def _register(M):
    ch = aa.ResidentChain()
    ch.reset()
    for L in M["layers"]:
        assert ch.layer(L["attn_norm"], L["post_norm"], L["mix"]) == 0, ch.last_error()
        m = L["moe"]
        ch.moe(m["router"], m["gate"], m["up"], m["down"], m["shg"], m["shu"], m["shd"], m["n_exp"], m["top_k"],
               m["intermed"], m["sgi"])
    dim = M["embed"].shape[1]
    ch.model(M["embed"], M["fnorm"], M["lm"], dim, M["vocab"])
    assert ch.ready(), f"chain not ready, last error {ch.last_error()}"
    return ch


def _close(got, want, what):
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    scale = float(np.max(np.abs(want)))
    err = float(np.max(np.abs(got.astype(np.float64) - want)))
    assert err <= CHAIN_RTOL * scale, f"{what}: max |err| {err:.3g} > {CHAIN_RTOL} x {scale:.3g}"


def _no_near_ties(routes, top_k, what):
    """The oracle's routing must not sit on a near-tie, or an f32 difference in the
    router logits could legitimately pick another expert (then change the seed)."""
    for i, (_, _, logits) in enumerate(routes):
        p = np.exp(logits.astype(np.float64) - logits.max())
        p = np.sort(p / p.sum())[::-1]
        if top_k < p.size:
            assert (p[top_k - 1] - p[top_k]) / p[top_k - 1] > 1e-3, f"{what}: layer {i} routing near a tie"


def _oracle_lanes(M, rows, n_layers=None, logits=True):
    out = [oracle.chain_forward(M, int(r), n_layers, logits) for r in rows]
    return out


def test_model_chain_layer_by_layer():
    """The residual stream after each layer, then the logits, against the oracle."""
    gen = synth.rng(2718)
    dim, inter, n_exp, top_k = 512, 256, 16, 4
    M = _chain_model(gen, dim, inter, n_exp, top_k, 1000, 40, SMALL_LAYERS)
    ch = _register(M)
    try:
        for row in (3, 37):
            for n in range(len(SMALL_LAYERS) + 1):
                H, _, routes = oracle.chain_forward(M, row, n, logits=False)
                _no_near_ties(routes, top_k, f"row {row}")
                _close(ch.hidden([row], n)[0], H, f"row {row} after {n} layers")
            _, want, _ = oracle.chain_forward(M, row)
            _close(ch.forward(row), want, f"row {row} logits")
    finally:
        ch.reset()


def test_model_chain_batch_lanes():
    """aspida_gpu_chain_forward_batch: every lane against the oracle and against its
    single-token forward (B = 2, 5 and 16: small-batch products, grouped experts over
    the lanes' tokens)."""
    gen = synth.rng(1618)
    dim, inter, n_exp, top_k = 512, 256, 16, 4
    M = _chain_model(gen, dim, inter, n_exp, top_k, 700, 64, SMALL_LAYERS)
    ch = _register(M)
    try:
        for B in (2, 5, 16):
            rows = gen.integers(0, 64, B).astype(np.int32)
            got = ch.forward_batch(rows)
            for b, r in enumerate(rows):
                _, want, routes = oracle.chain_forward(M, int(r))
                _no_near_ties(routes, top_k, f"B={B} lane {b}")
                _close(got[b], want, f"B={B} lane {b} (row {r})")
                _close(got[b], ch.forward(int(r)).astype(np.float64), f"B={B} lane {b} vs single")
            H = ch.hidden(rows, len(SMALL_LAYERS))
            for b, r in enumerate(rows):
                _close(H[b], oracle.chain_forward(M, int(r), logits=False)[0], f"B={B} lane {b} hidden")
    finally:
        ch.reset()


# Layers whose experts' combine takes the next norm at two lanes and more: a
# grouped matrix-core layer followed by one without a mixer (the combine forms
# the post-attention norm and the router reads it), that one followed by a
# mixer layer (the attention norm), and a last layer (the final norm).
FUSED_NORM_LAYERS = [
    (Q4, -1, (Q4, Q4, Q6, Q4, Q4, Q6), True),
    (None, -1, (Q4, Q4, Q6, Q4, Q4, Q6), True),
    (-1, Q4, (Q4, Q4, Q6, Q4, Q4, Q6), False),
]


def test_model_chain_norm_in_expert_combine():
    """Lane batches through layers whose experts' combine launch also adds the
    residual and forms the next norm: every lane's logits and residual stream
    against the oracle and against its single-token forward (which keeps the
    separate norm launches)."""
    gen = synth.rng(2718)
    dim, inter, n_exp, top_k = 512, 256, 16, 4
    M = _chain_model(gen, dim, inter, n_exp, top_k, 500, 64, FUSED_NORM_LAYERS)
    ch = _register(M)
    try:
        for B in (2, 8):
            rows = gen.integers(0, 64, B).astype(np.int32)
            got = ch.forward_batch(rows)
            for b, r in enumerate(rows):
                _, want, routes = oracle.chain_forward(M, int(r))
                _no_near_ties(routes, top_k, f"B={B} lane {b}")
                _close(got[b], want, f"B={B} lane {b} (row {r})")
                _close(got[b], ch.forward(int(r)).astype(np.float64), f"B={B} lane {b} vs single")
            for n in (1, 2, 3):
                H = ch.hidden(rows, n)
                for b, r in enumerate(rows):
                    _close(H[b], oracle.chain_forward(M, int(r), n_layers=n, logits=False)[0],
                           f"B={B} lane {b} hidden after {n} layers")
    finally:
        ch.reset()


def test_model_chain_graph_replay_matches_eager():
    """The first forward of a lane count runs eagerly and captures a graph; later ones
    replay it.  Replays, with eager work and synchronisation between them, give the
    eager results bit for bit."""
    gen = synth.rng(4669)
    dim, inter, n_exp, top_k = 512, 256, 16, 4
    M = _chain_model(gen, dim, inter, n_exp, top_k, 500, 32, SMALL_LAYERS[:2])
    ch = _register(M)
    try:
        ch.set_graphs(False)
        eager = {r: ch.forward(r) for r in (1, 9, 30)}
        eager_b = ch.forward_batch([4, 9, 1])
        ch.set_graphs(True)
        ch.begin()
        first = ch.forward(1)                  # eager run, then capture
        assert ch.graphs() == 1
        assert np.array_equal(first.view(np.uint32), eager[1].view(np.uint32))
        for rep in range(3):
            for r in (9, 30, 1):
                got = ch.forward(r)            # replay
                assert np.array_equal(got.view(np.uint32), eager[r].view(np.uint32)), f"replay {rep} row {r}"
            ch.hidden([r], 1)                  # eager work between replays
        for rep in range(3):
            got = ch.forward_batch([4, 9, 1])
            assert np.array_equal(got.view(np.uint32), eager_b.view(np.uint32)), f"batch replay {rep}"
        assert ch.graphs() >= 1
        ch.end()
        assert ch.graphs() == 0
        _, want, _ = oracle.chain_forward(M, 30)
        _close(eager[30], want, "row 30 logits")
    finally:
        ch.reset()


def test_model_chain_qwen3_moe_shapes():
    """Two layers at the Qwen3-30B-A3B MoE shape (dim 2048, 128 experts of 768, top-8,
    Q4_K gate/up and Q6_K down, gated shared expert, Q4_K 2048 x 2048 mixer), one lane
    and eight lanes."""
    gen = synth.rng(1234)
    dim, inter, n_exp, top_k = 2048, 768, 128, 8
    layers = [(Q4, -1, (Q4, Q4, Q6, Q4, Q4, Q6), True)] * 2
    M = _chain_model(gen, dim, inter, n_exp, top_k, 2048, 16, layers)
    ch = _register(M)
    try:
        want = {r: oracle.chain_forward(M, r) for r in range(8)}
        for r in (0, 5):
            _no_near_ties(want[r][2], top_k, f"row {r}")
            _close(ch.hidden([r], 2)[0], want[r][0], f"row {r} hidden")
            _close(ch.forward(r), want[r][1], f"row {r} logits")
        got = ch.forward_batch(np.arange(8, dtype=np.int32))
        for r in range(8):
            _no_near_ties(want[r][2], top_k, f"lane {r}")
            _close(got[r], want[r][1], f"lane {r} logits")
    finally:
        ch.reset()


def test_model_chain_rejects_bad_rows_and_registrations():
    gen = synth.rng(99)
    dim, inter, n_exp, top_k = 256, 256, 4, 2
    M = _chain_model(gen, dim, inter, n_exp, top_k, 300, 8, SMALL_LAYERS[:1])
    ch = _register(M)
    try:
        ch.last_error()
        y = ch.forward(8)                      # row out of range
        assert np.all(np.isnan(y)) and ch.last_error() != 0
        y = ch.forward_batch([0, -1])
        assert np.all(np.isnan(y)) and ch.last_error() != 0
        ok = ch.forward(7)
        assert np.all(np.isfinite(ok)) and ch.last_error() == 0
        # a routed tensor too short for n_exp experts: the chain is no longer ready
        L = M["layers"][0]
        m = L["moe"]
        assert ch.layer(L["attn_norm"], L["post_norm"], L["mix"]) == 0
        short = (m["gate"][0][: m["gate"][0].size // 2], m["gate"][1])
        ch.moe(m["router"], short, m["up"], m["down"], m["shg"], m["shu"], m["shd"], n_exp, top_k, inter, m["sgi"])
        assert not ch.ready() and ch.last_error() != 0
    finally:
        ch.reset()
    assert not ch.ready()
