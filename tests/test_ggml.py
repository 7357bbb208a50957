"""The GGML MUL_MAT boundary's host logic, checked on the CPU: GGML's type
traits for this path's types, the work-buffer size of ggml_graph_plan, and
every GGML_ASSERT of ggml_compute_forward_mul_mat turned into an error return
before anything is launched (fake device pointers are never dereferenced)."""
from __future__ import annotations

import pytest

from weft_amd import ggml as G
from weft_amd import _lib

INVALID, NOT_SUPPORTED = 1, 801  # hipErrorInvalidValue, hipErrorNotSupported

# ggml.c type_traits: (blck_size, type_size); ggml-cpu.c type_traits_cpu vec_dot_type
TRAITS = {G.F32: (1, 4, -1), G.Q4_0: (32, 18, G.Q8_0), G.Q8_0: (32, 34, -1),
          G.Q4_K: (256, 144, G.Q8_K), G.Q8_K: (256, 292, -1), G.IQ2_XXS: (256, 66, G.Q8_K),
          G.MXFP4: (32, 17, G.Q8_0), G.Q6_K: (256, 210, G.Q8_K), G.Q5_K: (256, 176, G.Q8_K),
          G.NVFP4: (64, 36, G.Q8_0), G.Q4_1: (32, 20, G.Q8_1), G.Q8_1: (32, 36, -1),
          G.IQ2_XS: (256, 74, G.Q8_K)}


def test_type_traits_follow_ggml():
    for t, (blck, size, vdt) in TRAITS.items():
        assert (G.blck_size(t), G.type_size(t), G.vec_dot_type(t)) == (blck, size, vdt)
        assert G.row_size(t, 4096) == size * 4096 // blck
    assert G.row_size(G.Q4_K, 100) == 0  # not whole blocks (ggml_row_size asserts)
    for other in (1, 6, 11, 41, 99):  # F16, Q5_0, Q3_K, past the enum, unknown
        assert (G.type_size(other), G.blck_size(other), G.vec_dot_type(other)) == (0, 0, -1)


def test_default_strides_are_ggml_new_tensor_strides():
    t = G.tensor(G.Q4_K, (4096, 11008, 2))
    assert list(t.ne) == [4096, 11008, 2, 1]
    assert list(t.nb) == [144, 2304, 2304 * 11008, 2304 * 11008 * 2]


def test_work_size_is_the_graph_plan_size():
    # ggml_row_size(vec_dot_type, nelements(src1)) (ggml-cpu.c:2819-2826)
    for t, (blck, size, vdt) in TRAITS.items():
        if vdt < 0:
            continue
        src0 = G.tensor(t, (4096, 64))
        src1 = G.tensor(G.F32, (4096, 7, 3, 2))
        assert G.mul_mat_work_size(src0, src1) == G.row_size(vdt, 4096 * 7 * 3 * 2)
        assert G.mul_mat_work_size(src0, G.tensor(vdt, (4096, 7))) == 0


def call(src0, src1, dst, wdata=1 << 30, wsize=1 << 30):
    with pytest.raises(_lib.HipError) as e:
        G.mul_mat(src0, src1, dst, wdata, wsize)
    assert _lib.load().weft_hip_get_last_error() == 0  # cleared by mul_mat
    return e.value.code


def ok_args(t=G.Q4_K, k=512, n=64, m=4, planes=(1, 1), bplanes=(1, 1)):
    return (G.tensor(t, (k, n, *planes), data=1 << 20),
            G.tensor(G.F32, (k, m, *bplanes), data=2 << 20),
            G.tensor(G.F32, (n, m, *bplanes), data=3 << 20))


def test_asserts_become_invalid_value():
    s0, s1, d = ok_args()
    assert call(s0, G.tensor(G.F32, (256, 4), data=2 << 20), d) == INVALID        # ne00 != ne10
    assert call(s0, s1, G.tensor(G.F32, (63, 4), data=3 << 20)) == INVALID        # ne0 != ne01
    assert call(s0, s1, G.tensor(G.F32, (64, 5), data=3 << 20)) == INVALID        # ne1 != ne11
    s0b, s1b, db = ok_args(planes=(2, 1), bplanes=(3, 1))                          # ne12 % ne02
    assert call(s0b, s1b, db) == INVALID
    bad = G.tensor(G.Q4_K, (512, 64), data=1 << 20, nb=[145, 288 + 2, 0, 0])      # nb00 != type size
    assert call(bad, s1, d) == INVALID
    xt = G.tensor(G.F32, (512, 4), data=2 << 20, nb=[8, 4096, 0, 0])             # nb10 != 4
    assert call(s0, xt, d) == INVALID
    dt = G.tensor(G.F32, (64, 4), data=3 << 20, nb=[4, 2, 8, 8])                  # nb0 > nb1
    assert call(s0, s1, dt) == INVALID
    assert call(G.tensor(G.Q4_K, (500, 64), data=1 << 20), G.tensor(G.F32, (500, 4), data=2 << 20),
                d) == INVALID                                                     # not whole blocks
    need = G.mul_mat_work_size(s0, s1)
    assert call(s0, s1, d, wsize=need - 1) == INVALID                              # work buffer short
    assert call(s0, s1, d, wdata=0) == INVALID
    assert call(s0, s1, d, wdata=(1 << 30) + 2) == INVALID                         # misaligned wdata


def test_types_outside_the_path_are_not_supported():
    s0, s1, d = ok_args()
    assert call(G.tensor(6, (512, 64), data=1 << 20, nb=[22, 352, 0, 0]), s1, d) == NOT_SUPPORTED  # Q5_0
    assert call(s0, G.tensor(G.Q8_0, (512, 4), data=2 << 20), d) == NOT_SUPPORTED  # not Q4_K's vec_dot type
    assert call(s0, s1, G.tensor(G.Q8_K, (64, 4), data=3 << 20, nb=[4, 256, 1024, 1024])) == NOT_SUPPORTED
    # a quantized src1 is read in place: its rows must be packed records
    q = G.tensor(G.Q8_K, (512, 4), data=2 << 20, nb=[292, 1024, 4096, 4096])
    assert call(s0, q, d) == NOT_SUPPORTED


def test_empty_product_launches_nothing():
    s0, _, _ = ok_args()
    G.mul_mat(s0, G.tensor(G.F32, (512, 0), data=2 << 20), G.tensor(G.F32, (64, 0), data=3 << 20))
    assert _lib.load().weft_hip_get_last_error() == 0


# ---------------------------------------------------------------- MUL_MAT_ID
def moe_args(t=G.Q4_K, k=512, n=64, n_as=8, n_ids=4, ne11=1, n_tok=3):
    return (G.tensor(t, (k, n, n_as), data=1 << 20),
            G.tensor(G.F32, (k, ne11, n_tok), data=2 << 20),
            G.tensor(G.I32, (n_ids, n_tok), data=4 << 20),
            G.tensor(G.F32, (n, n_ids, n_tok), data=3 << 20))


def test_mul_mat_id_work_size_is_the_graph_plan_size():
    # ggml-cpu.c:2827-2845 with CACHE_LINE_SIZE 64 and 8-byte row mappings
    s0, s1, ids, _ = moe_args(n_as=8, n_ids=4, ne11=1, n_tok=3)
    want = G.row_size(G.Q8_K, 512 * 3) + 8 + 8 * 8 + 8 + 8 * 4 * 3 * 8 + 8 + 64 * 8 + 64
    assert G.mul_mat_id_work_size(s0, s1, ids) == want
    q = G.tensor(G.Q8_K, (512, 1, 3))
    assert G.mul_mat_id_work_size(s0, q, ids) == want - G.row_size(G.Q8_K, 512 * 3) - 8


def call_id(s0, s1, ids, d, wdata=1 << 30, wsize=1 << 30):
    with pytest.raises(_lib.HipError) as e:
        G.mul_mat_id(s0, s1, ids, d, wdata, wsize)
    assert _lib.load().weft_hip_get_last_error() == 0
    return e.value.code


def test_mul_mat_id_asserts_become_invalid_value():
    s0, s1, ids, d = moe_args()
    f32_ids = G.tensor(G.F32, (4, 3), data=4 << 20)
    assert call_id(s0, s1, f32_ids, d) == INVALID                                  # ids not I32
    assert call_id(s0, s1, G.tensor(G.I32, (4, 2), data=4 << 20), d) == INVALID   # ids ne1 != tokens
    assert call_id(s0, G.tensor(G.F32, (512, 3, 3), data=2 << 20), ids,
                   G.tensor(G.F32, (64, 4, 3), data=3 << 20)) == INVALID          # n_ids % ne11
    assert call_id(s0, s1, ids, G.tensor(G.F32, (64, 3, 3), data=3 << 20)) == INVALID  # dst ne1
    assert call_id(G.tensor(G.Q4_K, (512, 64, 8, 2), data=1 << 20), s1, ids, d) == INVALID  # 4-d src0
    assert call_id(s0, s1, ids, d, wsize=G.row_size(G.Q8_K, 512 * 3) - 1) == INVALID
    assert call_id(G.tensor(6, (512, 64, 8), data=1 << 20, nb=[22, 352, 352 * 64, 0]), s1, ids,
                   d) == NOT_SUPPORTED
