"""CPU checks of the batch-1 launch planner (aspida_kq_matvec_plan): the
workgroup shape each decode and benchmark shape gets on a 256-CU MI355X.

The planner runs on the host, so these need no GPU (without one the library
assumes MI355X's 256 CUs).  Each row is a choice measured on MI355X; the
comment names the measurement it rests on.  The tuple is (matrix cores, waves
per workgroup, workgroups per 64-row tile, columns per wave, columns one after
another, 16-row workgroups).
"""
import pytest

import aspida_amd as aa

# (kind, in_dim, out_dim, plan)
PLANS = [
    # Llama-3-8B decode
    (aa.Q6_K, 4096, 6144, (True, 16, 1, 1, False, True)),     # q|k+v pair (planned as Q6_K): 6.0 us vs 6.3 on 8 waves
    (aa.Q4_K, 4096, 4096, (True, 16, 1, 1, False, True)),     # o: 16-row 4.3 us vs 5.8 on 64-row
    (aa.Q4_K, 4096, 28672, (True, 4, 1, 4, True, False)),     # gate|up: whole tiles of 4 waves, 4 columns each
    (aa.Q6_K, 14336, 4096, (True, 14, 1, 4, True, True)),     # down: 14 waves of 4 columns, one block per CU
    (aa.Q6_K, 4096, 128256, (True, 8, 1, 2, True, True)),     # head: 66 us vs 68 on 64-row in the decode step
    # Llama-3-70B decode
    (aa.Q6_K, 8192, 10240, (True, 8, 4, 1, False, False)),    # q|k+v pair: split columns over 4 workgroups
    (aa.Q4_K, 8192, 8192, (True, 8, 1, 4, True, True)),       # o: 9.2 us on 8 waves vs 10.1 on 16
    (aa.Q4_K, 8192, 57344, (True, 8, 1, 4, True, True)),      # gate|up: 16-row, 2-4% under 64-row
    (aa.Q6_K, 28672, 8192, (True, 8, 1, 14, True, True)),     # down: 35.7 us on 8 waves vs 36.8 on 16
    (aa.Q6_K, 8192, 128256, (True, 8, 1, 4, True, True)),     # head: rows of 32 blocks, 16-row
    # K-quant table (Llama-3-8B FFN shapes)
    (aa.Q2_K, 4096, 14336, (True, 16, 1, 1, False, False)),   # a tile per workgroup, a column per wave
    (aa.Q2_K, 14336, 4096, (True, 14, 1, 4, False, True)),    # 16-row prefetching waves: 7.7 us vs 8.8 on 64-row
    (aa.Q3_K, 4096, 14336, (True, 16, 1, 1, False, False)),
    (aa.Q3_K, 14336, 4096, (True, 14, 1, 4, False, True)),    # 16-row prefetching waves: 9.8 us vs 10.3
    (aa.Q5_K, 4096, 14336, (True, 16, 1, 1, False, False)),
    (aa.Q5_K, 14336, 4096, (True, 14, 1, 4, True, True)),
    # Q2_K / Q3_K elsewhere (size sweep, 70B shapes)
    (aa.Q3_K, 4096, 8192, (True, 8, 1, 2, False, True)),      # 2 blocks per CU, 8 prefetching waves: 6.2 us vs 7.4
    (aa.Q2_K, 8192, 8192, (True, 8, 1, 4, False, True)),      # 7.9 us vs 8.7 on 64-row
    (aa.Q2_K, 8192, 57344, (True, 4, 1, 8, False, False)),    # tall: 4 prefetching waves, 33.7 us vs 34.6
    (aa.Q3_K, 8192, 57344, (True, 4, 8, 1, False, False)),    # tall: rows over 8 groups, 44.5 us vs 46.9
    (aa.Q3_K, 4096, 128256, (True, 4, 1, 4, True, False)),    # more than 4 tiles per CU: whole tiles
    (aa.Q2_K, 28672, 8192, (True, 4, 4, 7, False, False)),    # long rows: 19.5 us vs 22.2
    (aa.Q3_K, 28672, 8192, (True, 8, 14, 1, False, False)),   # long Q3_K rows keep one-column waves
]


@pytest.fixture(scope="module")
def dev():
    aa.load()
    return aa.DeviceOps()


@pytest.mark.parametrize("kind,in_dim,out_dim,plan", PLANS,
                         ids=[f"{aa.KIND_NAMES[k]}-{o}x{i}" for k, i, o, _ in PLANS])
def test_decode_shape_plans(kind, in_dim, out_dim, plan, dev):
    assert dev.matvec_plan(kind, in_dim, out_dim) == plan


def test_vector_engine_switch_leaves_the_matrix_cores(dev):
    """aspida_kq_set_mv_engine(1) sends every kind to the vector-ALU kernels."""
    dev.set_mv_engine(1)
    try:
        assert not dev.matvec_plan(aa.Q4_K, 4096, 4096)[0]
    finally:
        dev.set_mv_engine(0)
    assert dev.matvec_plan(aa.Q4_K, 4096, 4096)[0]


def test_overrides_are_per_thread(dev):
    """The aspida_kq_set_* overrides change only the calling thread's launches:
    a thread that forces 64-row workgroups and the vector engine sees its own
    plans change, while this thread keeps the built-in ones."""
    import threading

    seen = {}

    def other():
        dev.set_mfma_rows(1)
        seen["rows"] = dev.matvec_plan(aa.Q4_K, 4096, 4096)
        dev.set_mv_engine(1)
        seen["engine"] = dev.matvec_plan(aa.Q4_K, 4096, 4096)[0]

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["rows"][5] is False and seen["rows"][0]   # 64-row workgroups in that thread
    assert seen["engine"] is False                         # vector engine in that thread
    assert dev.matvec_plan(aa.Q4_K, 4096, 4096) == (True, 16, 1, 1, False, True)  # untouched here
