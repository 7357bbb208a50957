"""End-to-end through weft_amd.runtime (the weft.runtime mirror) on the GPU:
device Buffers from torch tensors, shape inference, JIT reuse, and the
reference's native_jit repro case (examples/repro/weft/native_jit.py:52-79:
one Q4_0 / Q8_0 block replicated x8, K = 256, against the vec_dot oracle)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as o
from weft_amd import kernels as K
from weft_amd.runtime import Buffer, CompileOptions, compile, jit

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch, torch.device("cuda:0")


def test_jit_q4_k_decode_with_device_buffers(torch_dev):
    torch, dev = torch_dev
    n, k, m = 1024, 4096, 1
    w = o.quantize("q4_k", o.seeded_normal(61, (n, k), 0.02))
    x = o.seeded_normal(62, (m, k))
    W = Buffer(torch.from_numpy(w).to(dev), shape=(n, k), encoding="Q4_K")
    xq_t = torch.zeros(m * (k // 256) * 292, dtype=torch.uint8, device=dev)
    Xq = Buffer(xq_t, shape=(m, k), encoding="Q8_K")
    y_t = torch.zeros((m, n), dtype=torch.float32, device=dev)
    fn = jit(K.production_mul_mat_q4_k_decode)
    fn(W, torch.from_numpy(x).to(dev), Xq, y_t)
    want_xq = o.quantize("q8_k", x)
    assert np.array_equal(xq_t.cpu().numpy().reshape(m, -1), want_xq)
    e, a = o.mul_mat_f64("q4_k", w, want_xq, n, k, m)
    assert o.within_tolerance(y_t.cpu().numpy(), e, a).all()
    assert compile(K.production_mul_mat_q4_k_decode) is compile(K.production_mul_mat_q4_k_decode)


def test_native_jit_q4_0_replicated_block(torch_dev):
    torch, dev = torch_dev
    k = 256
    rng = np.random.default_rng(0x57454654)
    wb = o.quantize("q4_0", rng.standard_normal(32).astype(np.float32))
    xb = o.quantize("q8_0", rng.standard_normal(32).astype(np.float32))
    w, x = np.tile(wb, 8), np.tile(xb, 8)
    y_t = torch.zeros(1, dtype=torch.float32, device=dev)
    fn = compile(K.quantized_vec_dot_q4_0_q8_0)
    fn(Buffer(torch.from_numpy(w).to(dev), shape=(k,), encoding="Q4_0"),
       Buffer(torch.from_numpy(x).to(dev), shape=(k,), encoding="Q8_0"), y_t)
    want = o.vec_dot("q4_0", w, x, k)
    assert abs(float(y_t.item()) - want) <= 1e-4 + 2e-3 * abs(want)  # native_jit.py tolerance


def test_host_buffer_rejected_on_device(torch_dev):
    torch, dev = torch_dev
    fn = compile(K.row_dequantize_q4_k)
    w = torch.zeros(144, dtype=torch.uint8, device=dev)
    with pytest.raises(TypeError, match="host memory"):
        fn(Buffer(w, shape=(256,), encoding="Q4_K"), np.zeros(256, np.float32))


def test_jit_staged_prefill_with_the_reference_tuning_bindings(torch_dev):
    """production_mul_mat_q4_k_staged as weft-mul-mat.sh runs it: jit with the
    bindings of examples/kernels/mul_mat/tuning.json ("mul-mat:k1 q4_k
    prefill"), a second call reusing the artifact."""
    torch, dev = torch_dev
    n, k, m = 256, 1024, 80
    w = o.quantize("q4_k", o.seeded_normal(63, (n, k), 0.02))
    x = o.seeded_normal(64, (m, k))
    xq_t = torch.zeros(m * (k // 256) * 292, dtype=torch.uint8, device=dev)
    y_t = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
    options = CompileOptions(meta={"NC": 64, "KC": 512, "MC": 8, "MR": 2})
    fn = jit(K.production_mul_mat_q4_k_staged, options=options)
    args = (Buffer(torch.from_numpy(w).to(dev), shape=(n, k), encoding="Q4_K"),
            torch.from_numpy(x).to(dev), Buffer(xq_t, shape=(m, k), encoding="Q8_K"), y_t)
    fn(*args)
    fn(*args)
    assert compile(K.production_mul_mat_q4_k_staged, options=options) is fn.compiled
    want_xq = o.quantize("q8_k", x)
    assert np.array_equal(xq_t.cpu().numpy().reshape(m, -1), want_xq)
    e, a = o.mul_mat_f64("q4_k", w, want_xq, n, k, m)
    assert o.within_tolerance(y_t.cpu().numpy(), e, a).all()


@pytest.mark.parametrize("definition,fmt", [(K.production_mul_mat_q5_k, "q5_k"),
                                            (K.production_mul_mat_q4_k_staged, "q4_k")])
def test_tile_bindings_retile_the_gemv_launches(torch_dev, definition, fmt):
    """NC (weight rows per workgroup) and MR (activation rows per pass) reach
    the GEMV kernels: MR = 1 launches one pass per activation row, MR = 4 one
    per four; the outputs are bit-identical (each output is one wave's dot
    whatever the tiling) and within the oracle's bar."""
    from weft_amd import _lib
    torch, dev = torch_dev
    n, k, m = 300, 1024, 8  # M < 16: the GEMV path of every prefill entry point
    w = o.quantize(fmt, o.seeded_normal(65, (n, k), 0.02))
    x = o.seeded_normal(66, (m, k))
    outs, launches = [], []
    for meta in ({"NC": 7, "KC": 512, "MC": 8, "MR": 1, "NR": 2}, {"NC": 64, "KC": 512, "MC": 8, "MR": 4, "NR": 2}):
        fn = compile(definition, options=CompileOptions(meta=meta))
        assert dict(fn.metadata["bindings"]) == dict(sorted(meta.items()))
        xq_t = torch.zeros(m * (k // 256) * 292, dtype=torch.uint8, device=dev)
        y_t = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
        _lib.launch_log()
        fn(Buffer(torch.from_numpy(w).to(dev), shape=(n, k), encoding=fmt.upper()),
           torch.from_numpy(x).to(dev), Buffer(xq_t, shape=(m, k), encoding="Q8_K"), y_t)
        launches.append([name for name in _lib.launch_log() if "gemv" in name])
        outs.append(y_t.cpu().numpy())
        want_xq = o.quantize("q8_k", x)
        assert np.array_equal(xq_t.cpu().numpy().reshape(m, -1), want_xq)
        e, a = o.mul_mat_f64(fmt, w, want_xq, n, k, m)
        assert o.within_tolerance(outs[-1], e, a).all()
    assert len(launches[0]) == m and len(launches[1]) == m // 4, launches
    np.testing.assert_array_equal(outs[0], outs[1])
    assert _lib.load().weft_hip_set_tile_binding(b"NR", 2) == 0  # no GEMV knob


def test_tile_bindings_choose_the_q4k_gemm_tiling(torch_dev):
    """MC and NC reach the Q4_K prefill GEMM as its tile (activation rows x
    weight rows per workgroup tile, examples/kernels/mul_mat/q4_k_staged.py:
    20-24): each binding launches its own tiling and workgroup count (the
    launch log), and every tiling gives the same outputs bit for bit (each
    output is one wave's superblock chain in a fixed order) within the
    oracle's bar."""
    from weft_amd import _lib
    torch, dev = torch_dev
    n, k, m = 300, 1024, 80  # ragged tiles on both axes
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    w = o.quantize("q4_k", o.seeded_normal(67, (n, k), 0.02))
    x = o.seeded_normal(68, (m, k))
    want_xq = o.quantize("q8_k", x)
    e, a = o.mul_mat_f64("q4_k", w, want_xq, n, k, m)
    outs = []
    for mc, nc in ((64, 128), (32, 128), (64, 64), (32, 64), (8, 64)):
        fn = compile(K.production_mul_mat_q4_k_staged, options=CompileOptions(meta={"NC": nc, "KC": 512, "MC": mc, "MR": 2}))
        assert fn.metadata["bindings_without_launch_knob"] == ("KC",)
        xq_t = torch.zeros(m * (k // 256) * 292, dtype=torch.uint8, device=dev)
        y_t = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
        _lib.launch_log()
        fn(Buffer(torch.from_numpy(w).to(dev), shape=(n, k), encoding="Q4_K"),
           torch.from_numpy(x).to(dev), Buffer(xq_t, shape=(m, k), encoding="Q8_K"), y_t)
        gemm = [name for name in _lib.launch_log() if name.startswith("q4k_mfma_gemm")]
        mt, nt = (32 if mc <= 32 else 64), (64 if nc <= 64 else 128)
        tiles = -(-m // mt) * -(-n // nt)
        assert gemm == [f"q4k_mfma_gemm_{mt}x{nt}/{min(tiles, cus)}"], gemm
        assert np.array_equal(xq_t.cpu().numpy().reshape(m, -1), want_xq)
        outs.append(y_t.cpu().numpy())
        assert o.within_tolerance(outs[-1], e, a).all()
    for y in outs[1:]:
        np.testing.assert_array_equal(y.view(np.uint32), outs[0].view(np.uint32))


@pytest.mark.parametrize("definition,fmt", [(K.production_mul_mat_q5_k_decode, "q5_k"),
                                            (K.production_mul_mat_q6_k_decode, "q6_k"),
                                            (K.production_mul_mat_q4_1_decode, "q4_1")])
def test_tile_binding_nc_reaches_the_batch1_kernels(torch_dev, definition, fmt):
    """NC sets the weight rows per workgroup of the batch-1 kernels too:
    NC = 3 and NC = 200 give bit-identical rows (each one wave's dot)."""
    from weft_amd import _lib
    torch, dev = torch_dev
    n, k = 1000, 2048
    w = o.quantize(fmt, o.seeded_normal(67, (n, k), 0.02))
    x = o.seeded_normal(68, (1, k))
    act = o.ACT_OF[fmt]
    outs = []
    for nc in (3, 200):
        fn = compile(definition, options=CompileOptions(meta={"NC": nc}))
        xq_t = torch.zeros(o.record_bytes(act, k), dtype=torch.uint8, device=dev)
        y_t = torch.full((1, n), float("nan"), dtype=torch.float32, device=dev)
        _lib.launch_log()
        fn(Buffer(torch.from_numpy(w).to(dev), shape=(n, k), encoding=fmt.upper()),
           torch.from_numpy(x).to(dev), Buffer(xq_t, shape=(1, k), encoding=act.upper()), y_t)
        assert len(_lib.launch_log()) == 1
        outs.append(y_t.cpu().numpy())
        want_xq = o.quantize(act, x)
        e, a = o.mul_mat_f64(fmt, w, want_xq, n, k, 1)
        assert o.within_tolerance(outs[-1], e, a).all()
    np.testing.assert_array_equal(outs[0], outs[1])


def test_launch_log_stays_bounded_without_a_reader(torch_dev):
    """The launch log keeps nothing while off and at most its last 4096 bytes
    of names while on, however many launches go unread."""
    torch, _ = torch_dev
    from weft_amd import _lib
    lib = _lib.load()
    _lib.set_stream(torch.cuda.current_stream().cuda_stream)
    was = lib.weft_hip_set_launch_log(0)
    try:
        for _ in range(2000):
            lib.weft_hip_probe_empty()
        torch.cuda.synchronize()
        _lib.check("probe_empty")
        assert lib.weft_hip_launch_log(None, 0) == 0
        lib.weft_hip_set_launch_log(1)
        for _ in range(2000):
            lib.weft_hip_probe_empty()
        torch.cuda.synchronize()
        _lib.check("probe_empty")
        n = lib.weft_hip_launch_log(None, 0)
        assert 3000 < n <= 4096
        names = _lib.launch_log()
        assert names and set(names) == {"probe_empty_kernel"}
    finally:
        lib.weft_hip_set_launch_log(was)
