"""Pins the CPU oracle (oracle/kq_oracle.c) before it is trusted as the checker.

* F16_To_F32: all 65,536 half patterns against numpy's float16, with the
  exponent-31 -> +0.0 rule of src/llm/llm_dequant.adb:46-48.
* Decoders: bit-exact against the golden fixtures (tests/golden), whose values
  come from exact arithmetic over an independent restatement of the layouts,
  including the known-answer blocks of tests/test_kquant_synth.adb, and
  against the dequantizer of the reference's own GPU harness
  (gpu/test_matvec.cu:17-70, built into oracle/_ref/).
* QMatVec: against exact dot products, and the reference tests' invariant that
  the fused dot equals the dense dot of the dequantized row.
* LLM_Pool chunking, router and MoE: closed-form properties, brute force and
  tests/test_moe.adb's known answers.
"""
import numpy as np
import pytest

import oracle

KINDS = oracle.KQUANTS + (oracle.KIND_Q8_0,)
NAME = {0: "q4k", 1: "q6k", 2: "q5k", 3: "q3k", 4: "q2k", 5: "q80"}


def test_f16_exhaustive():
    got = oracle.f16_table()
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    exp31 = ((h >> 10) & 0x1F) == 31
    want[exp31] = 0.0
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # Inf/NaN read as +0.0 whatever the sign
    assert oracle.f16_to_f32(0x00, 0xFC) == 0.0 and np.signbit(np.float32(oracle.f16_to_f32(0x00, 0xFC))) == 0
    assert np.signbit(np.float32(oracle.f16_to_f32(0x00, 0x80)))  # -0.0 stays -0.0


@pytest.mark.parametrize("kind", KINDS)
def test_decode_known_answer_blocks(kind, golden):
    kat = golden("kq_kat.npz")
    blk = kat[f"{NAME[kind]}_block"]
    got = oracle.dequant(kind, blk, 256, 1)[0]
    assert np.array_equal(got.view(np.uint32), kat[f"{NAME[kind]}_expected"].view(np.uint32))


@pytest.mark.parametrize("kind", KINDS)
def test_decode_random_blocks_bit_exact(kind, golden):
    rnd = golden("kq_random.npz")
    blocks = rnd[f"{NAME[kind]}_blocks"]
    exp = rnd[f"{NAME[kind]}_expected"]
    got = oracle.dequant(kind, blocks.reshape(-1), 256 * blocks.shape[0], 1).reshape(exp.shape)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


@pytest.mark.parametrize("kind", oracle.KQUANTS)
def test_decode_matches_reference_harness(kind):
    """gpu/test_matvec.cu's own dequantizer, compiled from the reference tree."""
    if oracle.ref_lib() is None:
        pytest.skip("oracle/_ref not built (reference tree absent when build() ran)")
    gen = np.random.Generator(np.random.PCG64(99 + kind))
    for _ in range(400):
        blk = gen.integers(0, 256, oracle.BLOCK_BYTES[kind], dtype=np.uint8)
        ours = oracle.dequant(kind, blk, 256, 1)[0]
        ref = oracle.ref_deq_block(kind, blk)
        fin = np.isfinite(ref)   # the harness decodes Inf/NaN halves as Inf/NaN
        assert np.array_equal(ours[fin].view(np.uint32), ref[fin].view(np.uint32))


@pytest.mark.parametrize("kind", KINDS)
def test_qmatvec_known_answer_dot(kind, golden):
    """test_kquant_synth.adb: fused QMatVec == dense dot, |err| < 1e-4."""
    kat = golden("kq_kat.npz")
    y = oracle.qmatvec(kind, kat[f"{NAME[kind]}_block"], 256, 1, kat["x_pattern"])
    assert abs(float(y[0]) - float(kat[f"{NAME[kind]}_dot"])) < 1e-4


@pytest.mark.parametrize("kind", KINDS)
def test_qmatvec_exact_dot(kind, golden):
    mv = golden("kq_matvec.npz")
    out_dim, in_dim = mv[f"{NAME[kind]}_shape"]
    y = oracle.qmatvec(kind, mv[f"{NAME[kind]}_w"], int(in_dim), int(out_dim), mv[f"{NAME[kind]}_x"])
    err = np.abs(y.astype(np.float64) - mv[f"{NAME[kind]}_dot"])
    assert np.all(err <= 1e-6 * mv[f"{NAME[kind]}_mag"] + 1e-30)


@pytest.mark.parametrize("kind", oracle.KQUANTS)
def test_qmatvec_equals_dense_dot_of_dequant(kind):
    """test_qmatvec_q4k.adb:83 / test_q2k_real.adb:84: max abs < 1e-3."""
    from aspida_amd import synth
    gen = synth.rng(7 + kind)
    in_dim, out_dim = 1024, 37
    w = synth.weight_np(kind, out_dim, in_dim, gen)
    x = synth.activations_np(in_dim, gen)
    dense = oracle.dequant(kind, w, in_dim, out_dim).astype(np.float64) @ x.astype(np.float64)
    y = oracle.qmatvec(kind, w, in_dim, out_dim, x)
    assert np.max(np.abs(y - dense)) < 1e-3


def test_qmatvec_guards():
    w = np.zeros(144 * 4, np.uint8)
    with pytest.raises(ValueError):
        oracle.qmatvec(0, w, 300, 1, np.zeros(300, np.float32))     # in % 256 /= 0
    with pytest.raises(ValueError):
        oracle.qmatvec(0, w, 256, 1, np.zeros(255, np.float32))     # length mismatch


def test_qmatvec_threads_bitwise_equal():
    from aspida_amd import synth
    gen = synth.rng(3)
    w = synth.weight_np(0, 4096, 512, gen)
    x = synth.activations_np(512, gen)
    y1 = oracle.qmatvec(0, w, 512, 4096, x, nthreads=1)
    y8 = oracle.qmatvec(0, w, 512, 4096, x, nthreads=8)
    assert np.array_equal(y1.view(np.uint32), y8.view(np.uint32))


def test_pool_chunks():
    # serial below Min_Grain (llm_pool.adb:103-106)
    assert oracle.pool_chunks(1, 1024, 2048, 8) == [(1, 1024)]
    assert oracle.pool_chunks(1, 4096, 2048, 1) == [(1, 4096)]
    assert oracle.pool_chunks(1, 4096, 2048, 8) == [(1 + 512 * i, 512 * (i + 1)) for i in range(8)]
    for first, last, ncpu in ((1, 14336, 7), (5, 2052, 3), (1, 2049, 16), (1, 8, 8)):
        ch = oracle.pool_chunks(first, last, 2, ncpu)
        assert ch[0][0] == first and ch[-1][1] == last and len(ch) <= ncpu
        assert all(a[1] + 1 == b[0] for a, b in zip(ch, ch[1:]))
        sizes = [h - l + 1 for l, h in ch]
        assert max(sizes) == -(-(last - first + 1) // min(ncpu, last - first + 1))


def _route_fp64(logits, k):
    p = np.exp(logits.astype(np.float64) - logits.max())
    p /= p.sum()
    order = sorted(range(len(p)), key=lambda e: (-p[e], e))[:k]
    w = p[order] / p[order].sum()
    return np.array(order), w


@pytest.mark.parametrize("seed", range(5))
def test_route_matches_brute_force(seed):
    gen = np.random.Generator(np.random.PCG64(seed))
    logits = gen.standard_normal(128).astype(np.float32) * 3
    idx, w = oracle.route(logits, 8)
    ridx, rw = _route_fp64(logits, 8)
    assert np.array_equal(idx, ridx)
    assert np.allclose(w, rw, rtol=1e-5, atol=1e-7)


def test_route_ties_lowest_index():
    logits = np.zeros(16, np.float32)
    logits[[3, 9, 12]] = 2.0            # three-way tie at the top
    idx, w = oracle.route(logits, 4)
    assert idx.tolist() == [3, 9, 12, 0]
    idx, _ = oracle.route(np.zeros(8, np.float32), 3)
    assert idx.tolist() == [0, 1, 2]


@pytest.mark.parametrize("top_k", [2, 1])
def test_moe_known_answer(top_k, golden):
    """tests/test_moe.adb: Forward vs an independent recompute, tol 1e-4."""
    k = golden("moe_kat.npz")
    y, idx, _ = oracle.moe_forward(k["x"], 2, 2, 2, top_k, k["gate_inp"],
                                   (k["gate_exp"], -1), (k["up_exp"], -1), (k["down_exp"], -1),
                                   (k["sh_gate"], -1), (k["sh_up"], -1), (k["sh_down"], -1))
    assert idx.tolist() == k[f"idx_top{top_k}"].tolist()
    assert np.all(np.abs(y - k[f"expected_top{top_k}"]) < 1e-4)


def test_moe_kquant_matches_fp64_recompute():
    """K-quant experts: the oracle's Forward against an fp64 recompute over the
    oracle's own (golden-pinned) dequantized weights."""
    from aspida_amd import synth
    gen = synth.rng(11)
    dim, inter, n_exp, top_k = 512, 256, 6, 3
    gk, dk = 0, 1
    gate = synth.weight_np(gk, n_exp * inter, dim, gen)
    up = synth.weight_np(gk, n_exp * inter, dim, gen)
    down = synth.weight_np(dk, n_exp * dim, inter, gen)
    shg, shu = synth.weight_np(gk, inter, dim, gen), synth.weight_np(gk, inter, dim, gen)
    shd = synth.weight_np(dk, dim, inter, gen)
    router = (gen.standard_normal((n_exp, dim)) * 0.02).astype(np.float32)
    sgi = (gen.standard_normal(dim) * 0.02).astype(np.float32)
    x = synth.activations_np(dim, gen)
    y, idx, tw = oracle.moe_forward(x, dim, inter, n_exp, top_k, router, (gate, gk), (up, gk), (down, dk),
                                    (shg, gk), (shu, gk), (shd, dk), shared_gate_inp=sgi, nthreads=4)
    xd = x.astype(np.float64)
    G = oracle.dequant(gk, gate, dim, n_exp * inter).reshape(n_exp, inter, dim).astype(np.float64)
    U = oracle.dequant(gk, up, dim, n_exp * inter).reshape(n_exp, inter, dim).astype(np.float64)
    D = oracle.dequant(dk, down, inter, n_exp * dim).reshape(n_exp, dim, inter).astype(np.float64)
    ridx, rw = _route_fp64(router.astype(np.float64) @ xd, top_k)
    assert np.array_equal(idx, ridx)

    def ffn(g, u, d):
        a = g @ xd
        return d @ ((a / (1 + np.exp(-a))) * (u @ xd))
    want = sum(rw[i] * ffn(G[e], U[e], D[e]) for i, e in enumerate(ridx))
    sg = 1 / (1 + np.exp(-(sgi.astype(np.float64) @ xd)))
    want = want + sg * ffn(oracle.dequant(gk, shg, dim, inter).astype(np.float64),
                           oracle.dequant(gk, shu, dim, inter).astype(np.float64),
                           oracle.dequant(dk, shd, inter, dim).astype(np.float64))
    assert np.max(np.abs(y - want)) <= 1e-4 * np.max(np.abs(want))


def test_rmsnorm_closed_forms():
    """LLM_RMSNorm.Forward (llm_rmsnorm.adb:10-41): for x = c (constant) the
    output is c / sqrt(c^2 + 1e-6) * w -- at c = 1e-3 the epsilon halves the
    result, so a dropped or misplaced epsilon fails; for x = a e_j it is
    a / sqrt(a^2 / n + 1e-6) * w_j, which pins the mean (not the sum)."""
    gen = np.random.default_rng(5)
    for n in (256, 2048):
        w = (1 + 0.5 * gen.standard_normal(n)).astype(np.float32)
        for c in (3.0, 1e-3, -2.0):
            y = oracle.rmsnorm(np.full(n, c, np.float32), w)
            want = c / np.sqrt(np.float64(c) ** 2 + 1e-6) * w.astype(np.float64)
            assert np.allclose(y, want, rtol=2e-6, atol=0)
        x = np.zeros(n, np.float32)
        x[7] = 5.0
        y = oracle.rmsnorm(x, w)
        assert y[7] == pytest.approx(5.0 / np.sqrt(25.0 / n + 1e-6) * w[7], rel=2e-6)
        assert np.count_nonzero(y) == 1


def test_rmsnorm_matches_fp64():
    gen = np.random.default_rng(6)
    for n in (512, 4096):
        x = (gen.standard_normal(n) * 3).astype(np.float32)
        w = gen.standard_normal(n).astype(np.float32)
        xd = x.astype(np.float64)
        want = xd / np.sqrt(np.mean(xd * xd) + 1e-6) * w
        assert np.max(np.abs(oracle.rmsnorm(x, w) - want)) <= 1e-6 * np.max(np.abs(want))


def test_chain_forward_matches_fp64_recompute():
    """oracle.chain_forward against an fp64 recompute of the same model from the
    oracle's (golden-pinned) dequantized weights: per layer H += Mix norm(H) then
    H += MoE(norm(H)), then the head on the final norm (llm_qwen_blk.adb:125-170,
    llm_qwen.adb:1199-1203).  A residual added before its norm, a norm with the
    other layer weight or a missing residual all fail it."""
    from aspida_amd import synth
    gen = synth.rng(21)
    dim, inter, n_exp, top_k, vocab = 512, 256, 6, 2, 300
    gk, dk = 0, 1

    def mat(kind, out, inp):
        return synth.weight_np(kind, out, inp, gen), kind
    layers = []
    for li in range(2):
        layers.append({
            "attn_norm": (1 + 0.1 * gen.standard_normal(dim)).astype(np.float32),
            "post_norm": (1 + 0.1 * gen.standard_normal(dim)).astype(np.float32),
            "mix": mat(gk, dim, dim) if li == 0 else ((gen.standard_normal((dim, dim)) * 0.02).astype(np.float32), -1),
            "moe": {"router": ((gen.standard_normal((n_exp, dim)) * 0.1).astype(np.float32), -1) if li == 0
                    else mat(5, n_exp, dim),
                    "gate": mat(gk, n_exp * inter, dim), "up": mat(gk, n_exp * inter, dim),
                    "down": mat(dk, n_exp * dim, inter), "shg": mat(gk, inter, dim), "shu": mat(gk, inter, dim),
                    "shd": mat(dk, dim, inter), "sgi": (gen.standard_normal(dim) * 0.05).astype(np.float32),
                    "n_exp": n_exp, "top_k": top_k, "intermed": inter}})
    M = {"embed": gen.standard_normal((4, dim)).astype(np.float32),
         "fnorm": (1 + 0.1 * gen.standard_normal(dim)).astype(np.float32),
         "lm": mat(dk, vocab, dim), "vocab": vocab, "layers": layers}

    def deq(w, inp, out):
        arr, kind = w
        return (arr.reshape(out, inp) if kind == -1 else oracle.dequant(kind, arr, inp, out)).astype(np.float64)

    def norm(x, w):
        return x / np.sqrt(np.mean(x * x) + 1e-6) * w.astype(np.float64)

    def ffn(g, u, d, x):
        a = g @ x
        return d @ ((a / (1 + np.exp(-a))) * (u @ x))
    row = 2
    H = M["embed"][row].astype(np.float64)
    for L in layers:
        H = H + deq(L["mix"], dim, dim) @ norm(H, L["attn_norm"])
        m = L["moe"]
        nr = norm(H, L["post_norm"])
        ridx, rw = _route_fp64(deq(m["router"], dim, n_exp) @ nr, top_k)
        G = deq(m["gate"], dim, n_exp * inter).reshape(n_exp, inter, dim)
        U = deq(m["up"], dim, n_exp * inter).reshape(n_exp, inter, dim)
        D = deq(m["down"], inter, n_exp * dim).reshape(n_exp, dim, inter)
        y = sum(rw[i] * ffn(G[e], U[e], D[e], nr) for i, e in enumerate(ridx))
        sg = 1 / (1 + np.exp(-(m["sgi"].astype(np.float64) @ nr)))
        y = y + sg * ffn(deq(m["shg"], dim, inter), deq(m["shu"], dim, inter), deq(m["shd"], inter, dim), nr)
        H = H + y
    want = deq(M["lm"], dim, vocab) @ norm(H, M["fnorm"])
    got_h, got, routes = oracle.chain_forward(M, row)
    assert len(routes) == 2
    assert np.max(np.abs(got_h - H)) <= 1e-4 * np.max(np.abs(H))
    assert np.max(np.abs(got - want)) <= 1e-4 * np.max(np.abs(want))
    h1, none, _ = oracle.chain_forward(M, row, n_layers=0, logits=False)
    assert none is None and np.array_equal(h1, M["embed"][row])
