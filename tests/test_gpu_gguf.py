"""GPU: weights read from a GGUF file (aspida_amd.gguf) run through the packed
matvec and the reference's host-pointer matvec, against the oracle's QMatVec
on the same bytes -- the loader path a Q4_K_M model takes to the device
(src/llm/llm_weight.adb:115-131 reads ne0/ne1 and the data offset the same way)."""
import numpy as np
import pytest

import aspida_amd as aa
import oracle
from aspida_amd import gguf, synth
import gguf_writer as gw
from gpu_helpers import abs_dot_scale, assert_close_scaled, ncpu, stream, sync, to_dev, torch_cuda

pytestmark = pytest.mark.gpu

GGML = {aa.Q4_K: 12, aa.Q6_K: 14, aa.Q5_K: 13, aa.Q3_K: 11, aa.Q2_K: 10, aa.Q8_0: 8}
SHAPES = [("blk.0.attn_q.weight", aa.Q4_K, 4096, 1024), ("blk.0.attn_v.weight", aa.Q6_K, 4096, 1024),
          ("blk.0.ffn_down.weight", aa.Q6_K, 1536, 4096), ("blk.0.ffn_up.weight", aa.Q4_K, 4096, 300),
          ("blk.0.x5.weight", aa.Q5_K, 512, 640), ("blk.0.x3.weight", aa.Q3_K, 768, 130),
          ("blk.0.x2.weight", aa.Q2_K, 1024, 64), ("blk.0.x8.weight", aa.Q8_0, 2048, 200)]


def test_gguf_weights_on_device(tmp_path):
    torch = torch_cuda()
    dev = aa.DeviceOps()
    host = aa.LLMGpu()
    gen = synth.rng(90210)
    W = {n: synth.weight_np(k, out, inp, gen) for n, k, inp, out in SHAPES}
    path = tmp_path / "dev.gguf"
    gw.write(path, [(n, [inp, out], GGML[k], W[n].tobytes()) for n, k, inp, out in SHAPES],
             [("general.architecture", "str", "llama"), ("general.alignment", "u32", 256)], alignment=256)
    with gguf.GGUFFile(path) as g:
        assert g.alignment == 256
        for name, kind, inp, out in SHAPES:
            print(f"gguf tensor {name} kind {kind} {out}x{inp}", flush=True)
            packed, k, in_dim, out_dim = g.to_device_packed(dev, name)
            assert (k, in_dim, out_dim) == (kind, inp, out)
            x = synth.activations_np(inp, gen)
            dy = torch.empty(out, dtype=torch.float32, device="cuda")
            dev.matvec_packed(kind, packed.data_ptr(), inp, out, to_dev(x).data_ptr(), dy.data_ptr(), stream())
            sync()
            want = oracle.qmatvec(kind, W[name], inp, out, x, nthreads=ncpu())
            scale = abs_dot_scale(kind, W[name], inp, out, x)
            assert_close_scaled(dy.cpu().numpy(), want, scale, what=f"packed {name}")
            raw = np.array(g.weight(name)[0])
            assert raw.tobytes() == W[name].tobytes()
            y = host.matvec(raw, kind, inp, out, x)          # the Ada binding's entry point
            assert host.last_error() == 0
            assert_close_scaled(y, want, scale, what=f"host-pointer {name}")
            host.free_weight(raw)
