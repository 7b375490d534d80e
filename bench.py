#!/usr/bin/env python3
"""Benchmark of the quantized-weight hot path on one MI355X.

Workload (one "step" = one decoded token): the batch-1 weight stream of a
Llama-3-8B Q4_K_M model -- 32 layers of q, k, o, gate, up in Q4_K and v, down
in Q6_K, plus the Q6_K output head (4,875,853,824 weight bytes per token; the
Q4_K_M mix follows tools/probes/requantize.adb:103-113).  Each projection is a
fused dequant+dot matvec of libaspidagpu.so on weights resident in HBM, launched
in the decode order a layer needs them: q|k (one launch over the
concatenated rows) and v, then o, then the gate|up launch, then down; the
head at the end.  Weights sit in HBM in the library's packed layout (packed
once at load, as the drop-in ABI does on upload).  Attention, norms and SwiGLU
are not part of the path and are not run: their inputs are fixed synthetic
activations, so the step times only the quantized matvecs.  One step is
captured once in a HIP graph and replayed.

Printed: one JSON line (metric, value = tokens/s, roofline of the dominant
kernel measured with HIP events on its stream, cpu_baseline = the C oracle of
Aspida's CPU QMatVec on the host cores, the per-kind batch-1 matvec table
at the Llama-3-8B FFN shapes on cold HBM, the small-batch and MoE tables, the
same decode stream at Llama-3-70B shape: 80 layers, 44.4 GB per token, and the
resident model chain behind the reference chain ABI on a 48-layer
Qwen3-MoE-shaped model).
"""
import argparse
import json
import os
import statistics
import subprocess
import sys
import tempfile
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

HBM_PEAK_GBS = 8000.0
GIB = 1 << 30

# Llama-3-8B: hidden 4096, FFN 14336, 32 q heads / 8 kv heads of 128, vocab 128256.
HIDDEN, FFN, KV, VOCAB, LAYERS = 4096, 14336, 1024, 128256, 32
Q4_K, Q6_K = 0, 1
# The two weight streams: Llama-3-8B (the headline) and Llama-3-70B (hidden
# 8192, FFN 28672, 64 q heads / 8 kv heads of 128, 80 layers; 44.4 GB resident).
MODEL_8B = dict(name="llama3-8b", hidden=HIDDEN, ffn=FFN, kv=KV, vocab=VOCAB, layers=LAYERS,
                stream_bytes=4_875_853_824)
MODEL_70B = dict(name="llama3-70b", hidden=8192, ffn=28672, kv=1024, vocab=128256, layers=80,
                 stream_bytes=44_383_027_200)


def layer_plan(m=MODEL_8B):
    """(name, kind, out_dim, in_dim, input) per weight matrix of one layer."""
    h, f, kv = m["hidden"], m["ffn"], m["kv"]
    return [("qk", Q4_K, h + kv, h, "h"),
            ("v", Q6_K, kv, h, "h"),
            ("o", Q4_K, h, h, "att"),
            ("gate_up", Q4_K, 2 * f, h, "hn"),
            ("down", Q6_K, h, f, "act")]


# Rows of the batch-1 size sweep (out, in): 2 to 264 MB of Q4_K.
SWEEP_SHAPES = ((2048, 4096), (4096, 4096), (8192, 4096), (14336, 4096), (28672, 4096), (57344, 4096),
                (57344, 8192))


def size_sweep_table(torch, aa, synth, seed, stream):
    """Batch-1 matvec time against size per K-quant (SWEEP_SHAPES, cold HBM as
    kquant_table), and per kind the least-squares line t = t0 + bytes / R over
    the rows: t0 is the fixed cost of a launch (start-up, first loads, last
    column's arithmetic), R the rate at which the launch streams once running.
    A launch of b bytes reaches b / (t0 + b / R); "bytes_for_70pct" is the
    smallest size at which that is 70% of the HBM peak (null when R itself is
    below 70%)."""
    kinds = (aa.Q2_K, aa.Q3_K, aa.Q4_K, aa.Q5_K, aa.Q6_K)
    rows = kquant_table(torch, aa, synth, seed, stream,
                        shapes=[(k, o, i) for k in kinds for (o, i) in SWEEP_SHAPES])
    out = {"rows": rows, "fit": {}}
    for k in kinds:
        name = aa.KIND_NAMES[k]
        pts = [(aa.weight_bytes(k, i, o) + 4 * (i + o), rows[f"{name} {o}x{i}"]["us"] * 1e-6) for o, i in SWEEP_SHAPES]
        n = len(pts)
        mb, mt = sum(b for b, _ in pts) / n, sum(t for _, t in pts) / n
        slope = sum((b - mb) * (t - mt) for b, t in pts) / sum((b - mb) ** 2 for b, _ in pts)
        t0 = mt - slope * mb
        rate = 1.0 / slope / 1e9
        worst = max(abs(t - (t0 + slope * b)) for b, t in pts)
        p70 = 0.7 * HBM_PEAK_GBS * 1e9
        need = p70 * t0 / (1.0 - p70 * slope) if p70 * slope < 1.0 else None
        out["fit"][name] = {"t0_us": round(t0 * 1e6, 2), "stream_GBps": round(rate, 1),
                            "max_residual_us": round(worst * 1e6, 2),
                            "bytes_for_70pct": int(need) if need else None}
        print(f"# fit {name}: t0 {t0 * 1e6:.2f} us, streaming {rate:.0f} GB/s, max residual {worst * 1e6:.2f} us",
              file=sys.stderr, flush=True)
    return out


# Launches of one layer: q|k and v share their input and run as one launch.
LAYER_LAUNCHES = [("qk", "v"), ("o",), ("gate_up",), ("down",)]
# Token counts of the MoE prefill rows (the grouped-GEMM path from 96 tokens).
PREFILL_TOKENS = (128, 256, 512, 1024)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-table", action="store_true", help="skip the per-kind matvec table")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-threads", type=int, default=0, help="oracle threads (default min(16, cpus))")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--only", choices=["small", "moe", "kquant", "sweep", "decode70", "chain", "prefill", "abi",
                                       "resident", "warmcache"],
                    help="run just this table (no decode line): for profiling one workload; 'resident' times "
                         "the persistent matvec chain experiment beside the decode; 'warmcache' times the "
                         "decode's layer launches with their weights already in the Infinity Cache")
    ap.add_argument("--mv-engine", type=int, choices=[0, 1], default=0,
                    help="batch-1 engine: 0 = MFMA for Q4_K and Q6_K (default), 1 = the VALU kernel for every kind")
    ap.add_argument("--mm-engine", type=int, choices=[0, 1, 2, 3, 4, 5, 6], default=0,
                    help="small-batch engine for the 'small' table (aspida_kq_set_mm_engine): 0 = the library's pick")
    ap.add_argument("--no-70b", action="store_true", help="skip the Llama-3-70B weight-stream line")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="also run one device copy of this many MiB (calibrates rocprofv3 byte counters)")
    return ap.parse_args()


class Decoder:
    """Device-resident Llama-3 Q4_K_M weights (8B by default), in the packed
    layout of the batch-1 kernels, and the per-token launch list."""

    def __init__(self, torch, aa, synth, seed, engine=0, model=MODEL_8B):
        self.torch, self.dev = torch, aa.DeviceOps()
        self.aa = aa
        self.m = m = model
        self.engine = engine
        self.dev.set_mv_engine(engine)
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)

        def packed(kind, out, inp):
            raw = synth.blocks_torch(kind, out * (inp // 256), generator=g)
            p = torch.empty(self.dev.packed_bytes(kind, inp, out), dtype=torch.uint8, device="cuda")
            self.dev.pack(kind, raw.data_ptr(), inp, out, p.data_ptr())
            torch.cuda.synchronize()
            return p

        self.layers = [{name: packed(kind, out, inp) for name, kind, out, inp, _ in layer_plan(m)}
                       for _ in range(m["layers"])]
        self.head = packed(Q6_K, m["vocab"], m["hidden"])
        f = dict(device="cuda", dtype=torch.float32)
        hid = m["hidden"]
        self.x = {"h": torch.randn(hid, generator=g, **f), "att": torch.randn(hid, generator=g, **f),
                  "hn": torch.randn(hid, generator=g, **f), "act": torch.randn(m["ffn"], generator=g, **f)}
        self.y = {name: torch.empty(out, **f) for name, _, out, _, _ in layer_plan(m)}
        self.logits = torch.empty(m["vocab"], **f)

    def build_chain(self):
        """The whole token as one resident chain (aspida_kq_chain_*): per layer
        q|k and v read the layer input, o reads the q rows, gate|up reads o,
        down reads the gate rows, and the next layer reads down -- each step's
        input is the previous step's output, as in the decoder, with the
        element-wise work between them left out (it streams no weights).
        Outputs live in one arena, a vector per step and layer."""
        torch = self.torch
        plan = {name: (kind, out, inp) for name, kind, out, inp, _ in layer_plan()}
        sizes = [("h", HIDDEN)] + [(f"{n}{l}", plan[n][1]) for l in range(LAYERS) for n in plan] + [("logits", VOCAB)]
        off, n = {}, 0
        for name, size in sizes:
            off[name] = n
            n += (size + 63) // 64 * 64
        self.arena = torch.randn(n, device="cuda")
        base = self.arena.data_ptr()
        ptr = lambda name, start=0: base + 4 * (off[name] + start)
        steps = []
        for l, L in enumerate(self.layers):
            xin = ptr("h") if l == 0 else ptr(f"down{l - 1}")
            src = {"qk": xin, "v": xin, "o": ptr(f"qk{l}"), "gate_up": ptr(f"o{l}"), "down": ptr(f"gate_up{l}")}
            for name in ("qk", "v", "o", "gate_up", "down"):
                kind, out, inp = plan[name]
                steps.append((kind, L[name].data_ptr(), inp, out, src[name], ptr(f"{name}{l}")))
        steps.append((Q6_K, self.head.data_ptr(), HIDDEN, VOCAB, ptr(f"down{LAYERS - 1}"), ptr("logits")))
        self.chain_steps = steps
        self.chain = self.dev.chain(steps)
        return self.chain

    def launches(self):
        """Per launch, in decode order: a tuple of (kind, packed_ptr, in, out, x_key, y_ptr), one entry per
        matrix of the launch."""
        plan = {name: (kind, out, inp, xk) for name, kind, out, inp, xk in layer_plan(self.m)}
        for L in self.layers:
            for names in LAYER_LAUNCHES:
                yield tuple((plan[n][0], L[n].data_ptr(), plan[n][2], plan[n][1], plan[n][3], self.y[n].data_ptr())
                            for n in names)
        yield ((Q6_K, self.head.data_ptr(), self.m["hidden"], self.m["vocab"], "h", self.logits.data_ptr()),)

    def issue(self, op, stream):
        if len(op) == 1:
            kind, w, inp, out, xk, y = op[0]
            self.dev.matvec_packed(kind, w, inp, out, self.x[xk].data_ptr(), y, stream)
        else:
            (ka, wa, inp, oa, xk, ya), (kb, wb, _, ob, _, yb) = op
            self.dev.matvec2_packed(ka, wa, oa, ya, kb, wb, ob, yb, inp, self.x[xk].data_ptr(), stream)

    def step(self, stream, only=None):
        for op in self.launches():
            if only is None or only(op):
                self.issue(op, stream)


def mfma_walk(spw, seq):
    """The MFMA kernels' column-walk template argument: 0 one column per wave,
    1 prefetching waves, 2 columns one after another."""
    return 0 if spw == 1 else 2 if seq else 1


def kernel_name(dec, op):
    """The kernel symbol a launch runs: kq_mv_mfma<kind, waves, walk> and
    kq_mv_mfma2<kind_a, kind_b, waves, walk> (Q4_K and Q6_K on the matrix
    cores; kq_mv_mfma16 / kq_mv_mfma2_16 on 16-row workgroups),
    kq_mv_packed<kind, waves, prefetch> or
    kq_mv_packed2<kind_a, kind_b, waves, prefetch> (the launch split is the
    library's: aspida_kq_matvec_plan, aspida_kq_packed_plan)."""
    rows = sum(-(-o // 64) * 64 for _, _, _, o, _, _ in op)
    kinds = [m[0] for m in op]
    if len(op) == 1:
        mfma, nw, _, spw, seq, b16 = dec.dev.matvec_plan(kinds[0], op[0][2], rows)
        if mfma:
            return f"kq_mv_mfma{'16' if b16 else ''}<{kinds[0]}, {nw}, {mfma_walk(spw, seq)}>"
    else:
        aa = dec.aa
        # the pair runs on MFMA when both kinds do, with the wider kind's split
        mf = [dec.dev.matvec_plan(k, op[0][2], rows) for k in kinds]
        if all(m[0] for m in mf):
            _, nw, _, spw, seq, b16 = dec.dev.matvec_plan(aa.Q6_K if aa.Q6_K in kinds else kinds[0], op[0][2], rows)
            return f"kq_mv_mfma2{'_16' if b16 else ''}<{kinds[0]}, {kinds[1]}, {nw}, {mfma_walk(spw, seq)}>"
        nw, _, spw = dec.dev.packed_plan(op[0][2], rows)
    pf = "true" if spw > 1 else "false"
    kinds = ", ".join(str(m[0]) for m in op)
    return f"kq_mv_packed{'2' if len(op) > 1 else ''}<{kinds}, {nw}, {pf}>"


def op_bytes(aa, op):
    inp = op[0][2]
    return sum(aa.weight_bytes(kind, inp, out) + 4 * out for kind, _, _, out, _, _ in op) + 4 * inp


def kernel_events(torch, dec, stream, reps=5):
    """Per kernel symbol: the step's launches of that kernel alone, captured in
    a HIP graph and replayed `reps` times between two HIP events on the launch
    stream; average launch duration = elapsed / launches."""
    aa = dec.aa
    names = sorted({kernel_name(dec, op) for op in dec.launches()})
    out = {}
    for name in names:
        ops = [op for op in dec.launches() if kernel_name(dec, op) == name]
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            dec.step(stream.cuda_stream, only=lambda op: kernel_name(dec, op) == name)
        with torch.cuda.stream(stream):
            g.replay()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(reps):
                g.replay()
            e1.record(stream)
        stream.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        nbytes = sum(op_bytes(aa, op) for op in ops)
        out[name] = {"launches": len(ops), "us_per_step": round(us, 1),
                                        "avg_us": round(us / len(ops), 3), "bytes": nbytes,
                                        "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}
        del g
    return out


TRAFFIC_FILE = os.path.join(HERE, "profiles", "kq_mv_mfma_llama8b_decode_traffic.json")


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` in this workload, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE measurement (scaled by a copy kernel of
    known size); None when that file has no figure for the kernel."""
    try:
        with open(TRAFFIC_FILE) as f:
            k = json.load(f)["kernels"].get(kernel)
    except (OSError, ValueError, KeyError):
        return None
    return None if k is None else k["traffic_bytes_per_launch"]


def kquant_table(torch, aa, synth, seed, stream, shapes=None):
    """Batch-1 matvec per K-quant at the Llama-3-8B FFN shapes (and the 4096^2
    Q4_K q_proj), packed layout, rotating launches over >=1 GiB of distinct
    weight copies so every launch reads cold HBM; one graph of all copies,
    replayed.  `shapes`: (kind, out, in) rows instead of those."""
    dev = aa.DeviceOps()
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 1)
    if shapes is None:
        shapes = [(k, o, i) for k in (aa.Q2_K, aa.Q3_K, aa.Q4_K, aa.Q5_K, aa.Q6_K)
                  for (o, i) in ((14336, 4096), (4096, 14336))] + [(aa.Q4_K, 4096, 4096)]
    table = {}
    for kind, out, inp in shapes:
        pb = dev.packed_bytes(kind, inp, out)
        ncopy = max(8, -(-int(1.1 * GIB) // pb))
        raw = synth.blocks_torch(kind, out * (inp // 256), generator=g)
        P = torch.empty(ncopy * pb, dtype=torch.uint8, device="cuda")
        dev.pack(kind, raw.data_ptr(), inp, out, P.data_ptr())
        del raw
        for c in range(1, ncopy):   # copies at distinct addresses: caches are address-tagged, so each launch reads HBM
            P[c * pb:(c + 1) * pb].copy_(P[:pb])
        x = torch.randn(inp, device="cuda", generator=g)
        y = torch.empty(out, device="cuda")
        torch.cuda.synchronize()  # weights and x were written on the default stream
        with torch.cuda.stream(stream):
            sp = stream.cuda_stream
            dev.matvec_packed(kind, P.data_ptr(), inp, out, x.data_ptr(), y.data_ptr(), sp)
            stream.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for c in range(ncopy):
                    dev.matvec_packed(kind, P.data_ptr() + c * pb, inp, out, x.data_ptr(), y.data_ptr(),
                                      stream.cuda_stream)
            graph.replay()
            stream.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 4
            e0.record(stream)
            for _ in range(reps):
                graph.replay()
            e1.record(stream)
            stream.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / (reps * ncopy)
        nbytes = aa.weight_bytes(kind, inp, out) + 4 * (inp + out)
        gbs = nbytes / t / 1e9
        table[f"{aa.KIND_NAMES[kind]} {out}x{inp}"] = {"us": round(t * 1e6, 2), "GBps": round(gbs, 1),
                                                        "frac": round(gbs / HBM_PEAK_GBS, 3)}
        print(f"# {aa.KIND_NAMES[kind]} {out}x{inp}: {t * 1e6:.2f} us {gbs:.0f} GB/s", file=sys.stderr, flush=True)
        del graph, P
        torch.cuda.empty_cache()
    return table


def small_batch_table(torch, aa, synth, seed, stream, engine=0):
    """Small-batch products: Q4_K and Q6_K at 4096x4096 and
    14336x4096 for B in {2, 4, 8, 16, 32, 64}, packed weights (the library's
    pick per kind, shape and batch: small_batch_kernel), launches rotating
    over >= 1 GiB of weight copies.  GB/s counts W + 4 B (in + out) bytes;
    TFLOP/s counts 2 B in out."""
    dev = aa.DeviceOps()
    dev.set_mm_engine(engine)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 2)
    table = {}
    for kind in (aa.Q4_K, aa.Q6_K):
        for out, inp in ((4096, 4096), (14336, 4096)):
            pb = dev.packed_bytes(kind, inp, out)
            ncopy = max(8, -(-int(1.1 * GIB) // pb))
            raw = synth.blocks_torch(kind, out * (inp // 256), generator=g)
            P = torch.empty(ncopy * pb, dtype=torch.uint8, device="cuda")
            dev.pack(kind, raw.data_ptr(), inp, out, P.data_ptr())
            del raw
            for c in range(1, ncopy):
                P[c * pb:(c + 1) * pb].copy_(P[:pb])
            for B in (2, 4, 8, 16, 32, 64):
                X = torch.randn(B, inp, device="cuda", generator=g)
                Y = torch.empty(B, out, device="cuda")
                torch.cuda.synchronize()  # weights and X were written on the default stream
                with torch.cuda.stream(stream):
                    dev.matmul_packed(kind, P.data_ptr(), inp, out, B, X.data_ptr(), Y.data_ptr(), stream.cuda_stream)
                    stream.synchronize()
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph, stream=stream):
                        for c in range(ncopy):
                            dev.matmul_packed(kind, P.data_ptr() + c * pb, inp, out, B, X.data_ptr(), Y.data_ptr(),
                                              stream.cuda_stream)
                    graph.replay()
                    stream.synchronize()
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record(stream)
                    for _ in range(3):
                        graph.replay()
                    e1.record(stream)
                    stream.synchronize()
                t = e0.elapsed_time(e1) * 1e-3 / (3 * ncopy)
                nbytes = aa.weight_bytes(kind, inp, out) + 4 * B * (inp + out)
                table[f"{aa.KIND_NAMES[kind]} {out}x{inp} B={B}"] = {
                    "kernel": small_batch_kernel(aa, kind, inp, out, B) if engine == 0 else f"engine {engine}",
                    "us": round(t * 1e6, 2), "GBps": round(nbytes / t / 1e9, 1),
                    "hbm_frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 3),
                    "TFLOPs": round(2.0 * B * inp * out / t / 1e12, 2)}
                print(f"# {aa.KIND_NAMES[kind]} {out}x{inp} B={B}: {t * 1e6:.2f} us "
                      f"{nbytes / t / 1e9:.0f} GB/s", file=sys.stderr, flush=True)
                del graph
            del P
            torch.cuda.empty_cache()
    dev.set_mm_engine(0)
    return table


def small_batch_kernel(aa, kind, inp, out, B):
    """The kernel the library's default small-batch pick runs (mm_route in
    aspidagpu.hip) for Q4_K and Q6_K: up to 4 vectors the batch-1 kernel on
    4 vectors where the batch-1 plan is 16-row workgroups (and Q6_K at 2),
    else the one-pass kernel; the one-pass kernel up to 16 vectors and for
    Q6_K above (the wave-per-column kernel above 32 vectors on at most 1024
    (tile, column) pairs); Q4_K above 16 on the 64-vector MFMA kernel."""
    units = (-(-out // 64)) * (inp // 256)
    tall = units >= 8192
    if kind == aa.Q6_K and B > 32 and units <= 1024 and inp % 1024 == 0:
        return "kq_mmw"
    if B <= 4:
        if tall:
            return "kq_mv_mfma16n" if kind == aa.Q6_K else "kq_mm16_q4k"
        b16 = aa.DeviceOps().matvec_plan(kind, inp, out)[5]
        return "kq_mv_mfma16n" if b16 or (kind == aa.Q6_K and B <= 2) else "kq_mmv"
    if B <= 16 and tall:
        return "kq_mm16_q4k" if kind == aa.Q4_K else "kq_mm16_q6k"
    if B <= 16 or kind == aa.Q6_K:
        return "kq_mmv"
    return "kq_mm_mfma"


def moe_table(torch, aa, synth, seed, stream, tokens=(1, 8, 32), tag="MoE"):
    """Qwen3-MoE-style expert FFN: router f32 [128][2048],
    128 experts of gate/up Q4_K [768][2048] and down Q6_K [2048][768] plus one
    shared expert with a sigmoid gate, top-8, for T = 1, 8 and 32 tokens; the
    device path (router + grouped experts over packed expert tensors),
    rotating over three layers' weights (1.2 GB) so each layer reads cold HBM.
    GB/s counts the weights of the E_T distinct routed experts the router
    picked, the shared expert, the router and the activations; TFLOP/s counts
    2 T (top_k + 1) 3 dim I, the experts' multiply-adds (the prefill rows,
    `tokens` = 128 .. 1024, are compute-bound)."""
    dev = aa.DeviceOps()
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 3)
    dim, inter, n_exp, top_k, nlayers = 2048, 768, 128, 8, 3
    f = dict(device="cuda", dtype=torch.float32)
    sp0 = stream.cuda_stream

    def packed(kind, n, in_dim, out_dim):
        src = synth.blocks_torch(kind, n * out_dim * in_dim // 256, generator=g)
        dst = torch.empty(n * dev.packed_bytes(kind, in_dim, out_dim), dtype=torch.uint8, device="cuda")
        dev.pack_experts(kind, src.data_ptr(), src.numel() // n, in_dim, out_dim, n, dst.data_ptr(), sp0)
        stream.synchronize()
        del src
        return dst

    layers = []
    for _ in range(nlayers):
        layers.append({"router": torch.randn(n_exp, dim, generator=g, **f) * 0.02,
                       "sgi": torch.randn(dim, generator=g, **f) * 0.02,
                       "gate": packed(aa.Q4_K, n_exp, dim, inter), "up": packed(aa.Q4_K, n_exp, dim, inter),
                       "down": packed(aa.Q6_K, n_exp, inter, dim), "shg": packed(aa.Q4_K, 1, dim, inter),
                       "shu": packed(aa.Q4_K, 1, dim, inter), "shd": packed(aa.Q6_K, 1, inter, dim)})
    gs = aa.weight_bytes(aa.Q4_K, dim, inter)
    ds = aa.weight_bytes(aa.Q6_K, inter, dim)
    per_expert = 2 * gs + ds
    table = {}
    for T in tokens:
        X = torch.randn(T, dim, generator=g, **f)
        bufs = [{"logits": torch.empty(T, n_exp, **f), "idx": torch.empty(T, top_k, device="cuda", dtype=torch.int32),
                 "tw": torch.empty(T, top_k, **f),
                 "work": torch.empty(dev.moe_packed_work_bytes(T, dim, inter, top_k), dtype=torch.uint8,
                                     device="cuda"),
                 "y": torch.empty(T, dim, **f)} for _ in range(nlayers)]

        def run(sp):
            for L, B in zip(layers, bufs):
                dev.route(L["router"].data_ptr(), n_exp, dim, T, top_k, X.data_ptr(), B["logits"].data_ptr(),
                          B["idx"].data_ptr(), B["tw"].data_ptr(), sp)
                dev.moe_experts_packed(X.data_ptr(), T, dim, top_k, inter, n_exp, B["idx"].data_ptr(),
                                       B["tw"].data_ptr(), L["gate"].data_ptr(), L["up"].data_ptr(), aa.Q4_K,
                                       L["down"].data_ptr(), aa.Q6_K, L["shg"].data_ptr(), L["shu"].data_ptr(),
                                       L["shd"].data_ptr(), L["sgi"].data_ptr(), B["work"].data_ptr(),
                                       B["y"].data_ptr(), sp)

        torch.cuda.synchronize()  # weights and X were written on the default stream
        with torch.cuda.stream(stream):
            run(stream.cuda_stream)
            stream.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                run(stream.cuda_stream)
            graph.replay()
            stream.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 10
            e0.record(stream)
            for _ in range(reps):
                graph.replay()
            e1.record(stream)
            stream.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / (reps * nlayers)
        distinct = sum(len(set(B["idx"].cpu().numpy().ravel().tolist())) for B in bufs) / nlayers
        nbytes = (distinct + 1) * per_expert + n_exp * dim * 4 + 4 * T * (2 * dim)
        flops = 2.0 * T * (top_k + 1) * 3 * dim * inter
        table[f"T={T}"] = {"us": round(t * 1e6, 2), "distinct_experts": round(distinct, 1),
                           "GBps": round(nbytes / t / 1e9, 1), "hbm_frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 3),
                           "tok_s": round(T / t, 1), "TFLOPs": round(flops / t / 1e12, 2)}
        print(f"# {tag} T={T}: {t * 1e6:.2f} us, E_T={distinct:.1f}, {nbytes / t / 1e9:.0f} GB/s, "
              f"{flops / t / 1e12:.1f} TFLOP/s", file=sys.stderr, flush=True)
        del graph, bufs
    del layers
    torch.cuda.empty_cache()
    return table


def moe_chain_table(aa, synth, seed, tokens=20):
    """The resident model chain behind the reference's chain ABI
    (aspida_gpu_chain_moe / _model / _forward / _forward_batch,
    gpu_matvec.cu:2143-2400, 2783-2961) on a Qwen3-MoE-shaped model: 48 layers,
    each a Q4_K 2048 x 2048 matvec mixer (the stand-in for attention) and the
    config-3 MoE block (f32 router [128][2048], 128 experts of Q4_K gate/up
    [768][2048] and Q6_K down, a gated shared expert, top-8), then the Q6_K
    output head [151936][2048].  One layer's host weights are registered 48
    times: every layer gets its own copy in HBM (19 GB).  tok/s is end to end
    per forward call (row to the device, the graph replay, logits back to the
    host), at 1 lane and at 8 lanes (8 tokens per call)."""
    import numpy as np
    gen = synth.rng(seed + 11)
    dim, inter, n_exp, top_k, vocab, nlayers, rows = 2048, 768, 128, 8, 151936, 48, 1024
    ch = aa.ResidentChain()
    ch.reset()
    norm = (1.0 + 0.1 * gen.standard_normal(dim)).astype(np.float32)
    mix = (synth.weight_np(Q4_K, dim, dim, gen), Q4_K)
    router = ((gen.standard_normal((n_exp, dim)) * 0.02).astype(np.float32), -1)
    gate = (synth.weight_np(Q4_K, n_exp * inter, dim, gen), Q4_K)
    up = (synth.weight_np(Q4_K, n_exp * inter, dim, gen), Q4_K)
    down = (synth.weight_np(Q6_K, n_exp * dim, inter, gen), Q6_K)
    shg, shu = (synth.weight_np(Q4_K, inter, dim, gen), Q4_K), (synth.weight_np(Q4_K, inter, dim, gen), Q4_K)
    shd = (synth.weight_np(Q6_K, dim, inter, gen), Q6_K)
    sgi = (gen.standard_normal(dim) * 0.02).astype(np.float32)
    for _ in range(nlayers):
        assert ch.layer(norm, norm, mix) == 0
        ch.moe(router, gate, up, down, shg, shu, shd, n_exp, top_k, inter, sgi)
    ch.model(gen.standard_normal((rows, dim)).astype(np.float32), norm, (synth.weight_np(Q6_K, vocab, dim, gen), Q6_K),
             dim, vocab)
    assert ch.ready(), f"chain registration failed ({ch.last_error()})"
    del gate, up, down
    per_expert = 2 * aa.weight_bytes(Q4_K, dim, inter) + aa.weight_bytes(Q6_K, inter, dim)
    fixed = aa.weight_bytes(Q4_K, dim, dim) + n_exp * dim * 4     # mixer and router of a layer
    head = aa.weight_bytes(Q6_K, dim, vocab)
    out = {}
    for B in (1, 8):
        lanes = gen.integers(0, rows, (tokens + 1, B)).astype(np.int32)
        call = (lambda r: ch.forward(int(r[0]))) if B == 1 else (lambda r: ch.forward_batch(r))
        y = call(lanes[0])                                        # eager run, then the graph capture
        assert np.all(np.isfinite(y)) and ch.graphs() >= 1
        t0 = time.perf_counter()
        for r in lanes[1:]:
            call(r)
        t = (time.perf_counter() - t0) / tokens
        assert ch.last_error() == 0
        # Weight bytes per call: the experts the lanes' tokens touch are counted as
        # distinct per layer when B = 1 (top-8 + shared); for B lanes as the expected
        # number of distinct experts among B * 8 uniform picks (an estimate).
        distinct = top_k if B == 1 else n_exp * (1 - (1 - top_k / n_exp) ** B)
        nbytes = nlayers * (fixed + (distinct + 1) * per_expert) + head
        out[f"B={B}"] = {"tok_s": round(B / t, 1), "ms_per_call": round(t * 1e3, 3),
                         "weight_bytes_per_call": int(nbytes),
                         "hbm_frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 3)}
        print(f"# MoE chain B={B}: {B / t:.1f} tok/s, {t * 1e3:.3f} ms per call", file=sys.stderr, flush=True)
    ch.reset()
    out["model"] = {"layers": nlayers, "dim": dim, "experts": n_exp, "expert_ffn": inter, "top_k": top_k,
                    "shared_expert": True, "mixer": "Q4_K 2048x2048 matvec (stand-in for attention)",
                    "vocab": vocab, "head": "Q6_K", "tokens": tokens, "graph_replay": True}
    return out


def abi_path(aa, synth, seed, tokens=4):
    """The drop-in ABI as the reference's callers use it (LLM_GPU over
    aspida_gpu_matvec, gpu_matvec.cu:508-529): host x in, host y out, so each
    call pays its H2D of x, the kernel and its D2H of y.  Per K-quant at the
    two FFN shapes (median of repeated calls after the first, which mirrors
    the weight into HBM), and the 8B decode token as 32 x 7 calls plus the
    head over distinct host weights (4.9 GB, mirrored on the first token)."""
    import numpy as np
    gpu = aa.LLMGpu()
    gen = synth.rng(seed + 7)
    per_kind = {}
    for kind in (aa.Q2_K, aa.Q3_K, aa.Q4_K, aa.Q5_K, aa.Q6_K):
        for out, inp in ((14336, 4096), (4096, 14336)):
            w = synth.weight_np(kind, out, inp, gen)
            x = synth.activations_np(inp, gen)
            gpu.matvec(w, kind, inp, out, x)
            y = np.empty(out, np.float32)
            fn, args = gpu.lib.aspida_gpu_matvec, (w.ctypes.data, w.nbytes, kind, inp, out, x.ctypes.data,
                                                   y.ctypes.data)
            ts = []
            for _ in range(30):
                t0 = time.perf_counter()
                fn(*args)
                ts.append(time.perf_counter() - t0)
            assert gpu.last_error() == 0
            gpu.free_weight(w)
            t = statistics.median(ts)
            gbs = aa.weight_bytes(kind, inp, out) / t / 1e9
            per_kind[f"{aa.KIND_NAMES[kind]} {out}x{inp}"] = {"us": round(t * 1e6, 2), "weight_GBps": round(gbs, 1)}
    # The reference's seven calls per layer (q, k, v, o, gate, up, down).
    plan = [(Q4_K, HIDDEN, HIDDEN), (Q4_K, KV, HIDDEN), (Q6_K, KV, HIDDEN), (Q4_K, HIDDEN, HIDDEN),
            (Q4_K, FFN, HIDDEN), (Q4_K, FFN, HIDDEN), (Q6_K, HIDDEN, FFN)]
    layers = [[synth.weight_np(kind, out, inp, gen) for kind, out, inp in plan] for _ in range(LAYERS)]
    head = synth.weight_np(Q6_K, VOCAB, HIDDEN, gen)
    xs = {HIDDEN: synth.activations_np(HIDDEN, gen), FFN: synth.activations_np(FFN, gen)}

    # The calls with their arguments converted once, as a compiled caller
    # passes them (ctypes' per-call conversion of numpy buffers would add
    # about 5 us per call on the host, none of it the library's).
    ys = {n: np.empty(n, np.float32) for n in (HIDDEN, KV, FFN, VOCAB)}
    fn = gpu.lib.aspida_gpu_matvec
    calls_args = [(w.ctypes.data, w.nbytes, kind, inp, out, xs[inp].ctypes.data, ys[out].ctypes.data)
                  for ws in layers for (kind, out, inp), w in zip(plan, ws)]
    calls_args.append((head.ctypes.data, head.nbytes, Q6_K, HIDDEN, VOCAB, xs[HIDDEN].ctypes.data,
                       ys[VOCAB].ctypes.data))

    def token():
        for a in calls_args:
            fn(*a)

    token()                                          # mirrors every weight into HBM
    t0 = time.perf_counter()
    for _ in range(tokens):
        token()
    t_tok = (time.perf_counter() - t0) / tokens
    assert gpu.last_error() == 0
    for ws in layers:
        for w in ws:
            gpu.free_weight(w)
    gpu.free_weight(head)
    calls = LAYERS * len(plan) + 1
    print(f"# ABI path (host x/y per call): 8B decode {1 / t_tok:.1f} tok/s, {calls} calls/token", file=sys.stderr,
          flush=True)
    return {"decode_8b": {"tok_s": round(1 / t_tok, 2), "ms_per_token": round(t_tok * 1e3, 3),
                          "calls_per_token": calls, "tokens": tokens},
            "kquant_matvec": per_kind,
            "note": ("aspida_gpu_matvec with host buffers, synchronous: per call x is copied into pinned memory and "
                     "staged to HBM by a copy kernel that reads it, the matvec writes y straight into pinned host "
                     "memory, then the stream is synchronised (no copy-engine transfer per call)")}


def cpu_baseline(seed, threads, check_gpu=None):
    """Aspida's CPU QMatVec (restated in C, pooled rows as LLM_Pool does) on the
    same decode stream, timed on a bounded sample: one layer's seven matvecs
    (139 MB of weights) and the output head, each the median of repeated runs;
    tokens/s = 1 / (32 * layer + head).  With check_gpu = (torch, aa), the
    same weights and activations also run once through the decode's five GPU
    launch shapes and are checked against this QMatVec (gpu_spot_check)."""
    import numpy as np
    import oracle
    from aspida_amd import synth
    gen = synth.rng(seed)
    plan = [("q", Q4_K, HIDDEN, HIDDEN), ("k", Q4_K, KV, HIDDEN), ("v", Q6_K, KV, HIDDEN),
            ("o", Q4_K, HIDDEN, HIDDEN), ("gate", Q4_K, FFN, HIDDEN), ("up", Q4_K, FFN, HIDDEN),
            ("down", Q6_K, HIDDEN, FFN)]
    ws = [(kind, synth.weight_np(kind, out, inp, gen), inp, out) for _, kind, out, inp in plan]
    head = synth.weight_np(Q6_K, VOCAB, HIDDEN, gen)
    xs = {HIDDEN: synth.activations_np(HIDDEN, gen), FFN: synth.activations_np(FFN, gen)}

    def layer():
        for kind, w, inp, out in ws:
            oracle.qmatvec(kind, w, inp, out, xs[inp], nthreads=threads)

    def run_head():
        oracle.qmatvec(Q6_K, head, HIDDEN, VOCAB, xs[HIDDEN], nthreads=threads)

    def median_time(fn, budget_s, max_runs=60):
        fn(); fn()                                   # two warm-up calls
        ts, t_all = [], time.perf_counter()
        while len(ts) < max_runs and (len(ts) < 3 or time.perf_counter() - t_all < budget_s):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts), len(ts)

    t_layer, n_layer = median_time(layer, 12.0)
    t_head, n_head = median_time(run_head, 6.0)
    t_tok = LAYERS * t_layer + t_head
    parity = None
    if check_gpu is not None:
        named = {name: (kind, w) for (name, _, _, _), (kind, w, _, _) in zip(plan, ws)}
        parity = gpu_spot_check(*check_gpu, named, head, xs, threads)
        parity["small_batch"] = small_batch_spot_check(*check_gpu, named, gen, threads)
        parity["moe_layer"] = moe_spot_check(*check_gpu, gen, threads)
    return {"value": round(1.0 / t_tok, 4), "unit": "tok/s", "cores": threads, "kind": "port", "parity": parity,
            "sample": (f"C restatement of QMatVec (llm_dequant.adb:808-932, llm_pool.adb:91-160), "
                       f"{threads} threads; one Llama-3-8B layer's 7 matvecs (median of {n_layer}) and the "
                       f"Q6_K head (median of {n_head}); token = 32*layer + head = {t_tok * 1e3:.1f} ms; "
                       f"{(LAYERS * sum(w.nbytes for _, w, _, _ in ws) + head.nbytes) / t_tok / 1e9:.2f} GB/s"),
            "cpu_model": _cpu_model()}


def gpu_spot_check(torch, aa, named, head, xs, threads):
    """Ties the timed decode launches to the oracle: the CPU baseline's own
    Llama-3-8B layer and head, in the decode's launch shapes (q|k with v in one
    two-matrix launch, o, gate|up, down, head; the same entry points and
    therefore the same kernel picks as the timed token), computed once on the
    GPU and compared per output with QMatVec (llm_dequant.adb:808-932):
    |y - y_ref| <= 1e-4 * sum_i |w_i x_i|, ten times inside the 1e-3 bar.
    Returns the largest err / sum|w x| per launch; exits if any is out."""
    import numpy as np
    import oracle
    dev = aa.DeviceOps()
    cat = lambda a, b: (named[a][0], np.concatenate([named[a][1], named[b][1]]))
    mats = {"qk": cat("q", "k"), "v": named["v"], "o": named["o"], "gate_up": cat("gate", "up"),
            "down": named["down"], "head": (Q6_K, head)}
    dims = {"qk": (HIDDEN, HIDDEN + KV), "v": (HIDDEN, KV), "o": (HIDDEN, HIDDEN), "gate_up": (HIDDEN, 2 * FFN),
            "down": (FFN, HIDDEN), "head": (HIDDEN, VOCAB)}
    packed, ys = {}, {}
    for name, (kind, w) in mats.items():
        inp, out = dims[name]
        raw = torch.from_numpy(np.ascontiguousarray(w)).cuda()
        packed[name] = torch.empty(dev.packed_bytes(kind, inp, out), dtype=torch.uint8, device="cuda")
        dev.pack(kind, raw.data_ptr(), inp, out, packed[name].data_ptr())
        ys[name] = torch.empty(out, dtype=torch.float32, device="cuda")
    xd = {n: torch.from_numpy(np.ascontiguousarray(x)).cuda() for n, x in xs.items()}
    torch.cuda.synchronize()
    dev.matvec2_packed(Q4_K, packed["qk"].data_ptr(), HIDDEN + KV, ys["qk"].data_ptr(), Q6_K,
                       packed["v"].data_ptr(), KV, ys["v"].data_ptr(), HIDDEN, xd[HIDDEN].data_ptr())
    for name in ("o", "gate_up", "down", "head"):
        kind, _ = mats[name]
        inp, out = dims[name]
        dev.matvec_packed(kind, packed[name].data_ptr(), inp, out, xd[inp].data_ptr(), ys[name].data_ptr())
    torch.cuda.synchronize()
    worst = {}
    for name, (kind, w) in mats.items():
        inp, out = dims[name]
        want = oracle.qmatvec(kind, w, inp, out, xs[inp], nthreads=threads).astype(np.float64)
        scale = np.abs(oracle.dequant(kind, w, inp, out)).astype(np.float64) @ np.abs(xs[inp].astype(np.float64))
        err = np.abs(ys[name].cpu().numpy().astype(np.float64) - want) / np.maximum(scale, 1e-30)
        worst[name] = float(err.max())
        if not worst[name] <= 1e-4:
            print(f"bench.py: GPU decode launch '{name}' differs from the oracle: max err/sum|wx| "
                  f"{worst[name]:.3e} > 1e-4", file=sys.stderr, flush=True)
            sys.exit(1)
    return {"max_err_over_abs_dot": {k: float(f"{v:.3e}") for k, v in worst.items()}, "rtol": 1e-4,
            "launches": "q|k+v, o, gate|up, down, head on the baseline's own weights"}


def small_batch_spot_check(torch, aa, named, gen, threads):
    """Ties the small_batch table's kernels to the oracle: each small-batch
    kernel family the library picks at the table's shapes (small_batch_kernel)
    runs once through the same entry point (aspida_kq_matmul_packed_dev) --
    Q4_K 4096 x 4096 (the baseline's own o) at B = 2, 8 and 64, a Q6_K
    14336 x 4096 matrix at B = 2, 16 and 64 and a Q6_K 4096 x 4096 one at
    B = 64 -- and 64 sampled rows of every
    vector's output are compared with QMatVec (llm_dequant.adb:808-932) within
    1e-4 * sum_i |w_i x_i|.  Exits if any is out."""
    import numpy as np
    import oracle
    from aspida_amd import synth
    dev = aa.DeviceOps()
    q6 = synth.weight_np(Q6_K, FFN, HIDDEN, gen)
    q6s = synth.weight_np(Q6_K, HIDDEN, HIDDEN, gen)
    cases = [(Q4_K, named["o"][1], HIDDEN, HIDDEN, b) for b in (2, 8, 64)] + \
            [(Q6_K, q6, FFN, HIDDEN, b) for b in (2, 16, 64)] + [(Q6_K, q6s, HIDDEN, HIDDEN, 64)]
    worst = {}
    for kind, w, out, inp, B in cases:
        raw = torch.from_numpy(np.ascontiguousarray(w)).cuda()
        P = torch.empty(dev.packed_bytes(kind, inp, out), dtype=torch.uint8, device="cuda")
        dev.pack(kind, raw.data_ptr(), inp, out, P.data_ptr())
        X = synth.activations_np(B * inp, gen).reshape(B, inp)
        xd = torch.from_numpy(X).cuda()
        yd = torch.full((B, out), float("nan"), device="cuda")
        torch.cuda.synchronize()
        dev.matmul_packed(kind, P.data_ptr(), inp, out, B, xd.data_ptr(), yd.data_ptr())
        torch.cuda.synchronize()
        rows = np.sort(gen.choice(out, 64, replace=False))
        rb = aa.weight_bytes(kind, inp, 1)
        wr = np.ascontiguousarray(w.reshape(out, rb)[rows]).ravel()
        want = oracle.qmatmul(kind, wr, inp, rows.size, X, nthreads=threads).astype(np.float64)
        scale = np.abs(X.astype(np.float64)) @ np.abs(oracle.dequant(kind, wr, inp, rows.size)).astype(np.float64).T
        got = yd.cpu().numpy()[:, rows].astype(np.float64)
        err = float((np.abs(got - want) / np.maximum(scale, 1e-30)).max())
        name = f"{aa.KIND_NAMES[kind]} {out}x{inp} B={B} ({small_batch_kernel(aa, kind, inp, out, B)})"
        worst[name] = float(f"{err:.3e}")
        if not err <= 1e-4:
            print(f"bench.py: small batch {name} differs from the oracle: max err/sum|wx| {err:.3e} > 1e-4",
                  file=sys.stderr, flush=True)
            sys.exit(1)
        del P, raw
    return {"max_err_over_abs_dot": worst, "rtol": 1e-4, "rows_per_vector": 64}


def moe_spot_check(torch, aa, gen, threads):
    """Ties the moe_layer table's path to the oracle: the Qwen3-MoE layer shape
    (router f32 [128][2048], 128 experts of gate/up Q4_K [768][2048] and down
    Q6_K [2048][768], a gated shared expert, top-8) through the same device
    entry points as the table (aspida_moe_route_dev, then
    aspida_moe_experts_packed_dev) at T = 1, 8 and 32.  Per token: the GPU's
    expert choice equals the oracle's rule applied to the GPU's logits
    (llm_moe.adb:182-186), and the layer output equals the oracle's
    LLM_MoE.Forward experts (llm_moe.adb:111-302) on that choice within 1e-4
    of max |y|.  Exits if any is out."""
    import numpy as np
    import oracle
    from aspida_amd import synth
    dev = aa.DeviceOps()
    dim, inter, n_exp, top_k = 2048, 768, 128, 8
    gate = synth.weight_np(Q4_K, n_exp * inter, dim, gen)
    up = synth.weight_np(Q4_K, n_exp * inter, dim, gen)
    down = synth.weight_np(Q6_K, n_exp * dim, inter, gen)
    shg, shu = synth.weight_np(Q4_K, inter, dim, gen), synth.weight_np(Q4_K, inter, dim, gen)
    shd = synth.weight_np(Q6_K, dim, inter, gen)
    router = (gen.standard_normal((n_exp, dim)) * 0.02).astype(np.float32)
    sgi = (gen.standard_normal(dim) * 0.02).astype(np.float32)

    def packed(kind, w, n, in_dim, out_dim):
        src = torch.from_numpy(np.ascontiguousarray(w)).cuda()
        dst = torch.empty(n * dev.packed_bytes(kind, in_dim, out_dim), dtype=torch.uint8, device="cuda")
        dev.pack_experts(kind, src.data_ptr(), src.numel() // n, in_dim, out_dim, n, dst.data_ptr())
        return dst

    P = {"gate": packed(Q4_K, gate, n_exp, dim, inter), "up": packed(Q4_K, up, n_exp, dim, inter),
         "down": packed(Q6_K, down, n_exp, inter, dim), "shg": packed(Q4_K, shg, 1, dim, inter),
         "shu": packed(Q4_K, shu, 1, dim, inter), "shd": packed(Q6_K, shd, 1, inter, dim)}
    rd, sd = torch.from_numpy(router).cuda(), torch.from_numpy(sgi).cuda()
    worst = {}
    for T in (1, 8, 32):
        X = (gen.standard_normal((T, dim))).astype(np.float32)
        xd = torch.from_numpy(X).cuda()
        f = dict(device="cuda", dtype=torch.float32)
        logits, tw, y = torch.empty(T, n_exp, **f), torch.empty(T, top_k, **f), torch.empty(T, dim, **f)
        idx = torch.empty(T, top_k, device="cuda", dtype=torch.int32)
        work = torch.empty(dev.moe_packed_work_bytes(T, dim, inter, top_k), dtype=torch.uint8, device="cuda")
        torch.cuda.synchronize()
        dev.route(rd.data_ptr(), n_exp, dim, T, top_k, xd.data_ptr(), logits.data_ptr(), idx.data_ptr(),
                  tw.data_ptr())
        dev.moe_experts_packed(xd.data_ptr(), T, dim, top_k, inter, n_exp, idx.data_ptr(), tw.data_ptr(),
                               P["gate"].data_ptr(), P["up"].data_ptr(), Q4_K, P["down"].data_ptr(), Q6_K,
                               P["shg"].data_ptr(), P["shu"].data_ptr(), P["shd"].data_ptr(), sd.data_ptr(),
                               work.data_ptr(), y.data_ptr())
        torch.cuda.synchronize()
        L, I, W, Y = logits.cpu().numpy(), idx.cpu().numpy(), tw.cpu().numpy(), y.cpu().numpy()
        err = 0.0
        for t in range(T):
            ri, rw = oracle.route(L[t], top_k)
            if not (np.array_equal(ri, I[t]) and np.allclose(rw, W[t], rtol=1e-5, atol=1e-7)):
                print(f"bench.py: MoE T={T} token {t}: GPU routing {I[t]} differs from the oracle's rule on its "
                      f"logits {ri}", file=sys.stderr, flush=True)
                sys.exit(1)
            want = oracle.moe_experts(X[t], dim, top_k, inter, n_exp, I[t], W[t], (gate, Q4_K), (up, Q4_K),
                                      (down, Q6_K), (shg, Q4_K), (shu, Q4_K), (shd, Q6_K), sgi, nthreads=threads)
            err = max(err, float(np.abs(Y[t].astype(np.float64) - want).max() / max(np.abs(want).max(), 1e-30)))
        worst[f"T={T}"] = float(f"{err:.3e}")
        if not err <= 1e-4:
            print(f"bench.py: MoE layer T={T} differs from the oracle: max err / max|y| {err:.3e} > 1e-4",
                  file=sys.stderr, flush=True)
            sys.exit(1)
    return {"max_err_over_max_abs_y": worst, "rtol": 1e-4, "routing": "GPU choice == oracle rule on GPU logits"}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_cpus():
    """The host's CPUs as lscpu reports them, the CPUs this process may run on,
    and os.cpu_count()."""
    info = {"nproc": os.cpu_count(), "allowed": len(os.sched_getaffinity(0)), "model": _cpu_model()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        keys = {"Model name": "model", "CPU(s)": "cpus", "Socket(s)": "sockets", "Core(s) per socket":
                "cores_per_socket", "Thread(s) per core": "threads_per_core", "CPU max MHz": "max_mhz"}
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in keys:
                info[keys[k.strip()]] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return info


def native_oracle():
    """The oracle built -march=native for this host, at run time, into a
    temporary directory (the committed build is -march=x86-64-v3); None when
    no compiler is at hand."""
    src = os.path.join(os.path.dirname(os.path.abspath(__file__)), "oracle", "kq_oracle.c")
    out = os.path.join(tempfile.mkdtemp(prefix="oracle_native_"), "liboracle.so")
    cmd = ["gcc", "-O3", "-march=native", "-ffp-contract=off", "-fPIC", "-std=c11", "-shared", src, "-o", out,
           "-lm", "-lpthread"]
    try:
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    except (OSError, subprocess.SubprocessError):
        return None
    return out if r.returncode == 0 else None


def copy_probe(torch, mib):
    """One device-to-device copy of `mib` MiB: the known-size dispatch that
    calibrates FETCH_SIZE and WRITE_SIZE (aspida_amd.rocprof_summary
    --traffic --probe-kib)."""
    a = torch.empty(mib << 20, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    del a, b


def warm_cache_bound(torch, dec, stream, timed, tok_s, steps, warmup):
    """Experiment, not the headline: what the token would cost if every
    layer launch found its weights already in the caches.  The 32 layers'
    launches are issued over layer 0's weights (about 150 MB, inside the
    256 MB Infinity Cache, so after the first pass each launch reads cache),
    the head over its own (cold: 431 MB), in one graph timed as the decode
    is.  The gap to the cold token bounds what any scheme that fetches the
    next launch's weights ahead of it could gain."""
    ops = list(dec.launches())
    per_layer = len(LAYER_LAUNCHES)
    layer0, head = ops[:per_layer], ops[-1]
    nlayers = (len(ops) - 1) // per_layer

    def run(op_list):
        def fn(sp):
            for op in op_list:
                dec.issue(op, sp)
        wall, _ = timed(fn, steps, warmup)
        return wall / steps

    cold = run(ops)
    warm = run(layer0 * nlayers + [head])
    per_launch = {}
    for i, names in enumerate(LAYER_LAUNCHES):
        own = [ops[l * per_layer + i] for l in range(nlayers)]   # the 32 layers' copies of this launch
        per_launch["|".join(names)] = {"cold_us": round(run(own) * 1e6 / nlayers, 2),
                                       "warm_us": round(run([own[0]] * nlayers) * 1e6 / nlayers, 2)}
    return {"decode_tok_s": round(tok_s, 2), "token_cold_us": round(cold * 1e6, 1),
            "token_layers_warm_us": round(warm * 1e6, 1), "tok_s_cold": round(1 / cold, 1),
            "tok_s_layers_warm": round(1 / warm, 1), "per_launch": per_launch,
            "note": "the token's launches with the layers over layer 0's weights (cache-resident) against the "
                    "32 layers' own (HBM); the head is cold in both. per_launch: one launch kind, 32 in a graph, "
                    "over the 32 layers' weights (cold) or layer 0's (warm)"}


def timed_graph(torch, stream, step_fn, steps, warmup):
    """Capture one token, replay `warmup` times, then time `steps` replays
    (wall clock around synchronised replays, and HIP events on the stream)."""
    torch.cuda.synchronize()  # inputs were written on the default stream
    with torch.cuda.stream(stream):
        step_fn(stream.cuda_stream)
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step_fn(stream.cuda_stream)
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        e0.record(stream)
        for _ in range(steps):
            graph.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    del graph
    return wall, e0.elapsed_time(e1) * 1e-3


def decode_70b(torch, aa, synth, seed, stream, engine, steps, warmup):
    """the Llama-3-70B Q4_K_M decode weight stream, 44.4 GB
    of distinct resident weights per token, launched as the 8B stream is."""
    dec70 = Decoder(torch, aa, synth, seed + 70, engine, MODEL_70B)
    torch.cuda.synchronize()
    steps70 = max(5, min(steps, 20))
    w70, g70 = timed_graph(torch, stream, dec70.step, steps70, min(warmup, 3))
    b70 = MODEL_70B["stream_bytes"]
    big = {"workload": "llama3-70b-q4_k_m-decode-weight-stream", "layers": MODEL_70B["layers"],
           "hidden": MODEL_70B["hidden"], "ffn": MODEL_70B["ffn"], "kv_dim": MODEL_70B["kv"],
           "vocab": MODEL_70B["vocab"], "weight_bytes_per_token": b70, "steps": steps70,
           "tok_s": round(steps70 / w70, 2), "ms_per_step": round(w70 * 1e3 / steps70, 4),
           "gpu_event_ms_per_step": round(g70 * 1e3 / steps70, 4),
           "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / b70, 1),
           "hbm_frac_of_stream": round(steps70 / w70 * b70 / (HBM_PEAK_GBS * 1e9), 4)}
    print(f"# decode 70B (per-matrix launches): {big['tok_s']} tok/s "
          f"({big['hbm_frac_of_stream']:.3f} of the HBM roofline)", file=sys.stderr, flush=True)
    del dec70
    torch.cuda.empty_cache()
    return big


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the multi-GPU sharding is a design, not a measured path.", file=sys.stderr)
        sys.exit(2)
    import torch
    import aspida_amd as aa
    from aspida_amd import synth
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    aa.load()                                       # fails loudly without the HIP library
    stream = torch.cuda.Stream()
    if args.only == "decode70":
        print(json.dumps({"decode_70b": decode_70b(torch, aa, synth, args.seed, stream, args.mv_engine, args.steps,
                                                   args.warmup)}), flush=True)
        return
    if args.only and args.only not in ("resident", "warmcache"):
        if args.copy_probe_mib:
            copy_probe(torch, args.copy_probe_mib)
        if args.only == "abi":
            print(json.dumps({"abi_path": abi_path(aa, synth, args.seed)}), flush=True)
            return
        if args.only == "chain":
            print(json.dumps({"moe_chain": moe_chain_table(aa, synth, args.seed)}), flush=True)
            return
        if args.only == "prefill":
            print(json.dumps({"moe_prefill": moe_table(torch, aa, synth, args.seed, stream, PREFILL_TOKENS,
                                                        "MoE prefill")}), flush=True)
            return
        if args.only == "small":
            print(json.dumps({"small": small_batch_table(torch, aa, synth, args.seed, stream, args.mm_engine)}),
                  flush=True)
            return
        fn = {"moe": moe_table, "kquant": kquant_table, "sweep": size_sweep_table}[args.only]
        print(json.dumps({args.only: fn(torch, aa, synth, args.seed, stream)}), flush=True)
        return
    dec = Decoder(torch, aa, synth, args.seed, args.mv_engine)
    torch.cuda.synchronize()

    timed = lambda step_fn, steps, warmup: timed_graph(torch, stream, step_fn, steps, warmup)

    # The token: per-matrix launches of the packed batch-1 kernels (q|k and v
    # share one), captured in one HIP graph.
    wall, gpu_s = timed(dec.step, args.steps, args.warmup)
    tok_s = args.steps / wall
    print(f"# decode (per-matrix launches): {args.steps} tokens in {wall * 1e3:.1f} ms wall "
          f"({gpu_s * 1e3:.1f} ms events) = {tok_s:.1f} tok/s", file=sys.stderr, flush=True)
    if args.only == "warmcache":
        print(json.dumps({"warm_cache": warm_cache_bound(torch, dec, stream, timed, tok_s, args.steps,
                                                         args.warmup)}), flush=True)
        return
    if args.only == "resident":
        # Experiment, not the headline: the same token as one persistent
        # resident-chain launch (aspida_kq_chain_*), measured slower than the
        # per-matrix launches.
        chain = dec.build_chain()
        cwall, cgpu = timed(lambda sp: chain.run(sp), args.steps, args.warmup)
        chain_info = {"experiment": "persistent matvec chain (aspida_kq_chain_*)", "decode_tok_s": round(tok_s, 2),
                      "tok_s": round(args.steps / cwall, 2), "ms_per_step": round(cwall * 1e3 / args.steps, 4),
                      "gpu_event_ms_per_step": round(cgpu * 1e3 / args.steps, 4), "workgroups": chain.workgroups(),
                      "waits_completed": bool(chain.check())}
        chain.close()
        print(json.dumps({"resident_chain": chain_info}), flush=True)
        return

    # Dominant kernel: per kernel, its launches of one step in a graph of their own, timed with events.
    groups = kernel_events(torch, dec, stream)
    dom_key = max(groups, key=lambda k: groups[k]["us_per_step"])
    dom = groups[dom_key]
    achieved = dom["bytes"] / dom["launches"] / (dom["avg_us"] * 1e-6) / 1e9
    roofline = {"bound": "hbm", "kernel": dom_key, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom_key),
                "launches_per_step": dom["launches"], "avg_launch_us": dom["avg_us"],
                "bytes_per_launch": dom["bytes"] // dom["launches"]}
    stream_bytes = 4_875_853_824
    if args.copy_probe_mib:
        copy_probe(torch, args.copy_probe_mib)
    table = None if args.no_table else kquant_table(torch, aa, synth, args.seed, stream)
    small = None if args.no_table else small_batch_table(torch, aa, synth, args.seed, stream)
    moe = None if args.no_table else moe_table(torch, aa, synth, args.seed, stream)
    prefill = None if args.no_table else moe_table(torch, aa, synth, args.seed, stream, PREFILL_TOKENS, "MoE prefill")
    del dec
    torch.cuda.empty_cache()
    big = None if args.no_70b else decode_70b(torch, aa, synth, args.seed, stream, args.mv_engine, args.steps,
                                              args.warmup)

    abi = None if args.no_table else abi_path(aa, synth, args.seed)
    mchain = None if args.no_table else moe_chain_table(aa, synth, args.seed)

    cpu = None
    if not args.no_cpu:
        # This pool gives each GPU a share of 16 host CPUs; worker pools stay
        # within it whatever the node's CPU count (recorded in "host").
        host = host_cpus()
        threads = args.cpu_threads or min(16, host["allowed"] or 1)
        import oracle
        base = cpu_baseline(args.seed, threads, check_gpu=(torch, aa))
        builds = {"x86-64-v3": base["value"]}
        native = native_oracle()
        if native:
            oracle.use_library(native)
            nat = cpu_baseline(args.seed, threads)
            builds["native"] = nat["value"]
            if nat["value"] > base["value"]:
                base = {**nat, "parity": base["parity"]}
                base["sample"] += "; oracle built -march=native on this host at run time"
        cpu = {**base, "builds": builds, "host": host}
        print(f"# CPU baseline: {builds} tok/s on {threads} threads of {host.get('cpus', host['nproc'])} "
              f"({host.get('model', host['model'])})", file=sys.stderr, flush=True)

    line = {
        "metric": "Llama-3-8B Q4_K_M decode weight stream tok/s (batch 1) + K-quant matvec HBM GB/s",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "llama3-8b-q4_k_m-decode-weight-stream", "layers": LAYERS, "hidden": HIDDEN,
                   "ffn": FFN, "kv_dim": KV, "vocab": VOCAB, "batch": 1,
                   "weight_bytes_per_token": stream_bytes, "seed": args.seed},
        "hbm_frac_of_stream": round(tok_s * stream_bytes / (HBM_PEAK_GBS * 1e9), 4),
        "gpu_event_ms_per_step": round(gpu_s * 1e3 / args.steps, 4),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "abi_path": abi,
        "kernels": groups,
        "kquant_matvec": table,
        "small_batch": small,
        "moe_layer": moe,
        "moe_prefill": prefill,
        "moe_chain": mchain,
        "decode_70b": big,
    }
    assert dec_bytes_ok(MODEL_8B), "weight stream size drifted from the Llama-3-8B Q4_K_M layout"
    assert dec_bytes_ok(MODEL_70B), "weight stream size drifted from the Llama-3-70B Q4_K_M layout"
    print(json.dumps(line), flush=True)


def dec_bytes_ok(m):
    per_layer = sum({Q4_K: 144, Q6_K: 210}[k] * o * (i // 256) for _, k, o, i, _ in layer_plan(m))
    return m["layers"] * per_layer + 210 * m["vocab"] * (m["hidden"] // 256) == m["stream_bytes"]


if __name__ == "__main__":
    main()
