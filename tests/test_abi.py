"""The C ABI library loads, exports every symbol include/pdm.h declares, and
rejects bad arguments with a status code and message before touching a GPU."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    text = open(os.path.join(ROOT, "include", "pdm.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pdm_[a-z0-9_]+)\s*\(", text)))


def test_header_functions_match_binding_list(pdm):
    assert _header_functions() == sorted(pdm._lib.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(pdm):
    lib = pdm._lib.lib()
    for name in _header_functions():
        assert hasattr(lib, name), name
    assert lib.pdm_abi_version() == 10000


def test_struct_layouts_match_header(pdm):
    L = pdm._lib
    assert ctypes.sizeof(L.TableDesc) == 40
    assert ctypes.sizeof(L.BlockDesc) == 32
    assert ctypes.sizeof(L.BlockWeights) == 72
    assert L.SeqDesc.max_len.offset == 32
    assert ctypes.sizeof(L.SeqDesc) == 32 + 4 * 8 + 4 * 8 + 8 * 8 + 8 * 8
    assert ctypes.sizeof(L.OptimParams) == 40 and L.OptimParams.step.offset == 32


def test_argument_errors_are_reported_not_raised(pdm):
    L = pdm._lib
    lib = L.lib()
    h = ctypes.c_void_p()
    assert lib.pdm_tbe_plan_create(None, 1, ctypes.byref(h)) == L.PDM_ERR_INVALID
    assert "null" in L.last_error()
    bad = (L.TableDesc * 1)(L.TableDesc(10, 0, 6, L.PDM_F32, L.PDM_POOL_SUM, 0, 0, 0))
    assert lib.pdm_tbe_plan_create(bad, 1, ctypes.byref(h)) == L.PDM_ERR_INVALID
    assert "multiple of 4" in L.last_error()
    bad = (L.TableDesc * 1)(L.TableDesc(10, 0, 8, 9, L.PDM_POOL_SUM, 0, 0, 0))
    assert lib.pdm_tbe_plan_create(bad, 1, ctypes.byref(h)) == L.PDM_ERR_INVALID
    assert lib.pdm_tbe_pooled_fwd(None, None, None, 64, 0, None, 1, -1, None, 0, 8, None, None) == L.PDM_ERR_INVALID
    d = L.SeqDesc()
    d.num_pools = 0
    assert lib.pdm_seq_gather_fwd(ctypes.byref(d), None, None, None, None, None, None, None) == L.PDM_ERR_INVALID
    assert lib.pdm_int8_rowwise_quantize(None, 10, 0, None, 8, None) == L.PDM_ERR_INVALID
    one = (ctypes.c_int64 * 1)(1)
    assert lib.pdm_cross_hash_fwd(None, one, 1, 4, 10, 0, None, None) == L.PDM_ERR_INVALID
    assert "num_keys" in L.last_error()
    two = (ctypes.c_int64 * 2)(1, 1)
    assert lib.pdm_cross_hash_fwd(None, two, 2, 4, 0, 0, None, None) == L.PDM_ERR_INVALID
    assert "table_size" in L.last_error()
    assert lib.pdm_tbe_backward_workspace_size(None, 10, 2) == -1
    assert lib.pdm_tbe_plan_total_rows(None) == -1 and lib.pdm_tbe_plan_row_offset(None, 0) == -1
    assert lib.pdm_tbe_backward_fused(None, None, None, None, None, 64, 0, None, 1, -1, None, 8, None, None, 0,
                                      None, None) == L.PDM_ERR_INVALID
    assert "optimizer" in L.last_error()
    opt = L.OptimParams(L.PDM_OPT_ADAM, 0, 0.01, 1e-8, 0.9, 0.999, 0.0, 0, 1)
    assert lib.pdm_tbe_backward_fused(None, None, None, None, None, 64, 0, None, 1, -1, None, 8, ctypes.byref(opt),
                                      None, 0, None, None) == L.PDM_ERR_INVALID
    assert "null plan" in L.last_error()
    opt.optimizer = 7
    assert lib.pdm_tbe_backward_fused(None, None, None, None, None, 64, 0, None, 1, -1, None, 8, ctypes.byref(opt),
                                      None, 0, None, None) == L.PDM_ERR_INVALID
    assert lib.pdm_tbe_backward_sparse_grad(None, None, 64, 0, None, 1, -1, None, 8, None, None, None, None, 0, None,
                                            None) == L.PDM_ERR_INVALID
    assert "null plan" in L.last_error()


def test_ops_refuse_cpu_tensors(pdm):
    import torch

    with pytest.raises(RuntimeError, match="GPU only"):
        pdm.ops.int8_rowwise_quantize(torch.zeros(4, 8))
    with pytest.raises(RuntimeError, match="GPU only"):
        pdm.ops.seq_gather_raw([torch.zeros(4, 8, dtype=torch.bfloat16)], [[torch.zeros(1, dtype=torch.long)]],
                               [torch.zeros(2, dtype=torch.long)], [1])


def test_custom_ops_registered(pdm):
    import torch

    for name in ("tbe_pooled_fwd", "seq_gather_fwd", "onetrans_block_fwd", "onetrans_stack_fwd", "ec_lookup",
                 "tbe_fused_update", "ec_fused_update", "seq_fused_update", "kjt_permute", "cross_hash_fwd"):
        assert hasattr(torch.ops.pdm, name)


def test_block_workspace_size_matches_python_layout(pdm):
    L = pdm._lib
    for B, kv, q, ns, D, Fd in ((1024, 400, 272, 16, 256, 1024), (3, 33, 16, 16, 128, 384), (7, 9, 9, 0, 512, 128)):
        d = L.BlockDesc(B, D, D // 64, ns, Fd, kv, q, 0)
        got = L.lib().pdm_onetrans_block_workspace_size(ctypes.byref(d))
        assert got == pdm.ops.onetrans_workspace_layout(B, kv, q, D, Fd)["total"][0]
    bad = L.BlockDesc(4, 256, 2, 1, 1024, 10, 5, 0)  # head dim 128
    assert L.lib().pdm_onetrans_block_workspace_size(ctypes.byref(bad)) == L.PDM_ERR_INVALID
    assert "head dim" in L.last_error()
    bad = L.BlockDesc(4, 256, 4, 6, 1024, 10, 5, 0)  # q_len < n_ns
    assert L.lib().pdm_onetrans_block_workspace_size(ctypes.byref(bad)) == L.PDM_ERR_INVALID


def test_stack_workspace_size(pdm):
    """One block workspace for the largest layer (layer 0) plus two fp32 buffers of the largest inner layer's
    output; one buffer for two layers, none for one; schedules that grow or go negative are refused."""
    L = pdm._lib
    a = lambda v: (v + 255) // 256 * 256  # noqa: E731

    def size(B, kv, D, Fd, ns, q_s):
        d = L.BlockDesc(B, D, D // 64, ns, Fd, kv, 0, 0)
        arr = (ctypes.c_int32 * len(q_s))(*q_s)
        return L.lib().pdm_onetrans_stack_workspace_size(ctypes.byref(d), arr, len(q_s))

    B, kv, D, Fd, ns = 1024, 400, 256, 1024, 16
    block0 = pdm.ops.onetrans_workspace_layout(B, kv, 384 + ns, D, Fd)["total"][0]
    inner = a(B * (384 + ns) * D * 4)
    assert size(B, kv, D, Fd, ns, [384, 256, 128, 64]) == a(block0) + 2 * inner
    assert size(B, kv, D, Fd, ns, [384, 256]) == a(block0) + inner
    assert size(B, kv, D, Fd, ns, [384]) == a(block0)
    # the tiled path (d_model 384) holds h and g too: still layer 0's block workspace
    blk384 = pdm.ops.onetrans_workspace_layout(4, 60, 40 + 3, 384, 1536)["total"][0]
    assert size(4, 60, 384, 1536, 3, [40, 20]) == a(blk384) + a(4 * 43 * 384 * 4)
    assert size(B, kv, D, Fd, ns, [384, 390]) == L.PDM_ERR_INVALID  # layer 1 keeps more than its kv
    assert "q_len" in L.last_error()
    assert size(B, kv, D, Fd, ns, [384, -1]) == L.PDM_ERR_INVALID
    assert size(B, kv, D, Fd, ns, []) == L.PDM_ERR_INVALID
    d = L.BlockDesc(B, D, D // 64, ns, Fd, kv, 0, 0)
    assert L.lib().pdm_onetrans_stack_workspace_size(ctypes.byref(d), None, 2) == L.PDM_ERR_INVALID


def test_kjt_row_count_overflow_is_rejected(pdm):
    """num_features * batch_size (and num_out * batch_size) must be checked before the product is formed: a
    huge batch_size would otherwise wrap the int64 row count and pass the limits."""
    L = pdm._lib
    lib = L.lib()
    F = 64
    ids = (ctypes.c_void_p * F)(*([1] * F))
    lens = (ctypes.c_int32 * F)(*([4] * F))
    huge = 1 << 58
    assert lib.pdm_kjt_from_dense(ids, lens, F, huge, 64, 0, None, None, None, None, 0, None) == L.PDM_ERR_INVALID
    assert "overflow" in L.last_error()
    assert lib.pdm_kjt_from_dense_noalloc(ids, lens, F, huge, 64, 0, None, None, None, None) == L.PDM_ERR_INVALID
    assert "no-allocation limit" in L.last_error()
    assert lib.pdm_kjt_from_dense_noalloc(ids, lens, F + 1, 1, 64, 0, None, None, None, None) == L.PDM_ERR_INVALID
    assert "num_features" in L.last_error()
    perm = (ctypes.c_int32 * F)(*range(F))
    assert lib.pdm_kjt_permute(None, 64, None, F, huge, perm, F, None, None, None, None, 0, None) == L.PDM_ERR_INVALID
    assert "overflow" in L.last_error()
