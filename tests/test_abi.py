"""C-ABI and host-logic tests that run without a GPU.

They load libdsa_amd.so, check it exports every function include/dsa_abi.h
declares, and exercise the host-side validation paths, which all return
before anything is launched.
"""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest
import torch

from dsa_amd import _lib, workloads

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dsa_abi.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dsa_[a-z0-9_]+)\s*\(", text)))


def test_header_functions_are_exported():
    lib = _lib.load()
    declared = _declared_functions()
    assert declared, "no declarations parsed from dsa_abi.h"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in dsa_abi.h but not exported"
    assert set(declared) == set(_lib.EXPORTED_SYMBOLS)


def test_abi_version_and_struct_layout(tmp_path):
    """The ctypes mirrors match the C structs field by field (gcc offsetof)."""
    lib = _lib.load()
    assert lib.dsa_abi_version() == _lib.ABI_VERSION == 5
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "dsa_abi.h"', 'int main(void){']
    for cname, cls in (("dsa_attn_args", _lib.AttnArgs), ("dsa_indexer_args", _lib.IndexerArgs),
                        ("dsa_k_append_args", _lib.KAppendArgs),
                        ("dsa_indexer_k_prepare_args", _lib.KPrepareArgs)):
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for f, _ in cls._fields_:
            lines.append(f'printf("{cname}.{f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.check_call(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)])
    got = dict(l.split() for l in subprocess.check_output([str(exe)], text=True).splitlines())
    for cname, cls in (("dsa_attn_args", _lib.AttnArgs), ("dsa_indexer_args", _lib.IndexerArgs),
                        ("dsa_k_append_args", _lib.KAppendArgs),
                        ("dsa_indexer_k_prepare_args", _lib.KPrepareArgs)):
        assert int(got[cname]) == ctypes.sizeof(cls)
        for f, _ in cls._fields_:
            assert int(got[f"{cname}.{f}"]) == getattr(cls, f).offset, f


def test_split_choice():
    lib = _lib.load()
    assert lib.dsa_attn_num_splits(64, 16, 2048, 0) == 4       # decode fills 256 CUs
    # a workgroup takes chunks of up to 2048 keys
    assert lib.dsa_attn_num_splits(2048, 16, 2048, 0) == 1     # 2048-key chunks: prefill needs no split
    assert lib.dsa_attn_num_splits(256, 128, 2048, 0) == 1     # one-slice layout: 2048-key chunks
    assert lib.dsa_attn_num_splits(64, 128, 4096, 1) == 2      # ... and no longer
    assert lib.dsa_attn_num_splits(2048, 16, 1024, 0) == 1     # prefill needs no split
    assert lib.dsa_attn_num_splits(8, 16, 4096, 1) == 2        # requests below the minimum are raised
    # four-wave layout (H = 16 x odd, or x even while T x groups <= 128): the
    # most splits whose T x S x groups workgroups fit 256 CUs, at most 16,
    # >= one 16-key block per wave
    assert lib.dsa_attn_num_splits(1, 16, 2048, 0) == 16
    assert lib.dsa_attn_num_splits(16, 16, 2048, 0) == 16
    assert lib.dsa_attn_num_splits(32, 16, 2048, 0) == 8
    assert lib.dsa_attn_num_splits(8, 48, 2048, 0) == 10        # 24 x 10 = 240 workgroups
    assert lib.dsa_attn_num_splits(64, 48, 2048, 0) == 1
    assert lib.dsa_attn_num_splits(4, 16, 256, 0) == 4          # 64 keys per split
    assert lib.dsa_attn_num_splits(1, 16, 32768, 0) == 16       # 2048-key chunks at most
    assert lib.dsa_attn_num_splits(1, 32, 2048, 0) == 16
    assert lib.dsa_attn_num_splits(4, 128, 2048, 0) == 8        # 4 x 8 x 8 = 256
    # shared-ring layouts: one round of their workgroups
    assert lib.dsa_attn_num_splits(64, 128, 2048, 0) == 2       # 64 x 2 workgroups of 4 groups
    assert lib.dsa_attn_num_splits(128, 32, 2048, 0) == 2       # 2 groups x 4 slices
    assert lib.dsa_attn_num_splits(64, 16, 2048, 16) == 16     # explicit request honoured
    assert lib.dsa_attn_num_splits(1, 16, 5, 128) == 5         # at most one key per split
    assert lib.dsa_attn_num_splits(4, 16, 0, 0) == 1
    # fp32 partial outputs, then (max, sum) pairs
    assert lib.dsa_attn_workspace_bytes(64, 16, 2048, 0) == 64 * 4 * 16 * (512 + 16) * 4
    assert lib.dsa_attn_workspace_bytes(256, 128, 2048, 2) == 256 * 2 * 128 * 528 * 4
    assert lib.dsa_attn_workspace_bytes(2048, 16, 1024, 0) == 0
    # in-kernel merge (four-wave layout: odd numbers of 16-head groups): 8 wave
    # counters per (token, workgroup along the heads); other layouts use none
    assert lib.dsa_attn_counter_bytes(64, 16) == 64 * 8 * 4
    assert lib.dsa_attn_counter_bytes(4, 48) == 4 * 3 * 8 * 4    # 3 groups, one workgroup each
    assert lib.dsa_attn_counter_bytes(256, 128) == 0
    assert lib.dsa_attn_counter_bytes(8, 32) == 0
    assert lib.dsa_attn_counter_bytes(0, 16) == 0
    # per call: only calls that merge inside the kernel (2..4 splits, odd
    # group counts) use counters
    assert lib.dsa_attn_call_counter_bytes(64, 16, 2048, 0) == 64 * 8 * 4   # 4 splits
    assert lib.dsa_attn_call_counter_bytes(64, 16, 2048, 2) == 64 * 8 * 4
    assert lib.dsa_attn_call_counter_bytes(1, 16, 2048, 0) == 0             # 16 splits
    assert lib.dsa_attn_call_counter_bytes(48, 16, 2048, 5) == 0
    assert lib.dsa_attn_call_counter_bytes(64, 16, 2048, 1) == 0            # no split
    assert lib.dsa_attn_call_counter_bytes(2048, 16, 2048, 0) == 0
    assert lib.dsa_attn_call_counter_bytes(64, 128, 2048, 2) == 0           # even group count
    assert lib.dsa_attn_call_counter_bytes(4, 48, 2048, 3) == 4 * 3 * 8 * 4
    assert lib.dsa_attn_call_counter_bytes(4, 16, 2048, -1) == 0


def _args(**kw):
    a = _lib.AttnArgs()
    base = dict(q_nope=0x1000, q_nope_stride_t=16 * 512, q_nope_stride_h=512,
                q_pe=0x2000, q_pe_stride_t=16 * 64, q_pe_stride_h=64,
                ckv=0x3000, ckv_stride_page=64 * 512, ckv_stride_tok=512,
                kpe=0x4000, kpe_stride_page=64 * 64, kpe_stride_tok=64,
                sparse_indices=0x5000, idx_stride_t=2048,
                output=0x6000, out_stride_t=16 * 512, out_stride_h=512,
                lse=0x7000, lse_stride_t=16, lse_stride_h=1,
                num_tokens=64, num_heads=16, topk=2048, page_size=64, num_pages=2048,
                head_dim_ckv=512, head_dim_kpe=64, sm_scale=0.07, num_splits=0,
                workspace=None, workspace_bytes=0)
    base.update(kw)
    for k, v in base.items():
        setattr(a, k, v)
    return a


def _call(a):
    lib = _lib.load()
    rc = lib.dsa_attn_fwd(ctypes.byref(a), None)
    return rc, lib.dsa_last_error().decode()


@pytest.mark.parametrize("kw,code,needle", [
    (dict(head_dim_ckv=256), _lib.DSA_EUNSUPPORTED, "head dims"),
    (dict(num_heads=8), _lib.DSA_EUNSUPPORTED, "multiple of 16"),
    (dict(num_heads=0), _lib.DSA_EINVAL, "negative or zero"),
    (dict(page_size=0), _lib.DSA_EINVAL, "negative or zero"),
    (dict(num_splits=-1), _lib.DSA_EINVAL, "num_splits"),
    (dict(q_nope=None), _lib.DSA_EINVAL, "NULL"),
    (dict(ckv=0x3008), _lib.DSA_EINVAL, "16-byte"),
    (dict(q_nope_stride_h=500), _lib.DSA_EINVAL, "16-byte"),
    (dict(output=0x6002), _lib.DSA_EINVAL, "8-byte"),
    (dict(), _lib.DSA_EWORKSPACE, "workspace"),            # decode needs 4 splits
    (dict(num_splits=2, workspace=0x8000, workspace_bytes=16), _lib.DSA_EWORKSPACE, "workspace"),
    (dict(workspace=0x8000, workspace_bytes=1 << 30, split_counters=0x9000,
          split_counters_bytes=64), _lib.DSA_EWORKSPACE, "split_counters"),
    (dict(workspace=0x8000, workspace_bytes=1 << 30, split_counters=0x9002,
          split_counters_bytes=1 << 20), _lib.DSA_EWORKSPACE, "split_counters"),
])
def test_host_validation_rejects_before_launch(kw, code, needle):
    rc, msg = _call(_args(**kw))
    assert rc == code and needle in msg


def test_zero_tokens_is_a_no_op():
    rc, msg = _call(_args(num_tokens=0, q_nope=None))
    assert rc == _lib.DSA_OK and msg == ""


def test_null_args():
    lib = _lib.load()
    assert lib.dsa_attn_fwd(None, None) == _lib.DSA_EINVAL


def test_shim_rejects_cpu_tensors_and_bad_shapes():
    from dsa_amd import kernel
    d = workloads.cfg1()
    with pytest.raises(ValueError, match="GPU"):
        kernel(d["q_nope"], d["q_pe"], d["ckv_cache"], d["kpe_cache"], d["sparse_indices"],
               d["sm_scale"])
    with pytest.raises(ValueError, match="int32"):
        kernel(d["q_nope"], d["q_pe"], d["ckv_cache"], d["kpe_cache"],
               d["sparse_indices"].long(), d["sm_scale"])
    with pytest.raises(ValueError, match="multiple of 16"):
        kernel(d["q_nope"][:, :8], d["q_pe"][:, :8], d["ckv_cache"], d["kpe_cache"],
               d["sparse_indices"], d["sm_scale"])


def test_workload_generators_shapes_and_padding():
    d = workloads.cfg1()
    assert d["sparse_indices"].shape == (4, 256) and (d["sparse_indices"][3, 200:] == -1).all()
    assert (d["sparse_indices"][:3] >= 0).all()
    for row in d["sparse_indices"][:3]:
        assert row.unique().numel() == 256
    assert workloads.attention_bytes(d["sparse_indices"]) == (3 * 256 + 200) * 1152
    bt = torch.tensor([3, 0, 2, 1], dtype=torch.int32)
    pos = torch.tensor([[0, 5, 64, 130, -1]])
    assert workloads.positions_to_slots(pos, bt, 64).tolist() == [[192, 197, 0, 130, -1]]
    sel = workloads._distinct_below(1 << 17, 2048, torch.Generator().manual_seed(0))
    assert sel.unique().numel() == 2048 and int(sel.max()) < (1 << 17)
    assert np.isclose(workloads.SM_SCALE, 1 / np.sqrt(192))


def _idx_args(**kw):
    a = _lib.IndexerArgs()
    base = dict(q_idx=0x1000, k_idx=0x2000, k_scale=0x3000, weights=0x4000, causal_limit=0x5000,
                num_tokens=64, num_heads=64, head_dim=128, num_positions=32768, topk=2048,
                block_table=None, block_table_stride=0, page_size=64, out=0x6000,
                scores_out=None, workspace=0x8000,
                workspace_bytes=_lib.load().dsa_indexer_workspace_bytes(64, 64, 128, 32768))
    base.update(kw)
    for k, v in base.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,code,needle", [
    (dict(head_dim=64), _lib.DSA_EUNSUPPORTED, "head_dim"),
    (dict(num_heads=8), _lib.DSA_EUNSUPPORTED, "num_heads"),
    (dict(num_heads=128), _lib.DSA_EUNSUPPORTED, "num_heads"),
    (dict(topk=-1), _lib.DSA_EINVAL, "negative"),
    (dict(q_idx=None), _lib.DSA_EINVAL, "NULL"),
    (dict(out=None), _lib.DSA_EINVAL, "NULL"),
    (dict(k_idx=0x2008), _lib.DSA_EINVAL, "misaligned"),
    (dict(block_table=0x7000, page_size=0), _lib.DSA_EINVAL, "block_table"),
    (dict(workspace_bytes=1024), _lib.DSA_EWORKSPACE, "workspace"),
    (dict(k_cache=0x9000, k_pages=0xa000, k_page_size=64), _lib.DSA_EINVAL, "not both"),
    (dict(k_idx=None, k_scale=None, k_cache=0x9000, k_pages=None, k_page_size=64),
     _lib.DSA_EINVAL, "k_pages"),
    (dict(k_idx=None, k_scale=None, k_cache=0x9000, k_pages=0xa000, k_page_size=62),
     _lib.DSA_EINVAL, "multiple of 4"),
    (dict(k_idx=None, k_scale=None, k_cache=0x9008, k_pages=0xa000, k_page_size=64),
     _lib.DSA_EINVAL, "misaligned"),
    # every page a selected position can fall in must have a block-table entry
    (dict(block_table=0x7000, block_table_width=511), _lib.DSA_EINVAL, "block_table rows"),
    (dict(block_table=0x7000, block_table_width=512, block_table_stride=256),
     _lib.DSA_EINVAL, "below its width"),
    (dict(k_idx=None, k_scale=None, k_cache=0x9000, k_pages=0xa000, k_page_size=64),
     _lib.DSA_EINVAL, "k_num_pages"),
])
def test_indexer_host_validation(kw, code, needle):
    lib = _lib.load()
    rc = lib.dsa_indexer_topk(ctypes.byref(_idx_args(**kw)), None)
    assert rc == code and needle in lib.dsa_last_error().decode()


def test_indexer_workspace_and_empty_call():
    lib = _lib.load()
    # k operand chunks (3 pieces x 2 k-steps x 1 KB per 16 positions) + block
    # maxima, the per-position scales, fp32 scores; each region 256-aligned
    # (the q operands are derived inside the score kernel)
    def up(x):
        return (x + 255) // 256 * 256

    kb = 32768 // 16
    want = up(kb * 6144) + up(kb * 4) + up(32768 * 4) + up(64 * 32768 * 4)
    assert lib.dsa_indexer_workspace_bytes(64, 64, 128, 32768) == want
    kb = (1000 + 15) // 16
    want = up(kb * 6144) + up(kb * 4) + up(1000 * 4) + up(3 * 1000 * 4)
    assert lib.dsa_indexer_workspace_bytes(3, 48, 128, 1000) == want
    # with prepared K planes only the scores remain
    assert lib.dsa_indexer_workspace_bytes_prepared(3, 48, 128, 1000) == up(3 * 1000 * 4)
    assert lib.dsa_indexer_topk(ctypes.byref(_idx_args(num_tokens=0, q_idx=None)), None) == 0


def test_k_planes_sizes():
    """Prepared K planes hold exactly the K regions of a call's workspace: the
    k operand chunks, the block maxima and the per-position scales."""
    lib = _lib.load()

    def up(x):
        return (x + 255) // 256 * 256

    for S in (32768, 1000, 1, 0):
        kb = (S + 15) // 16
        assert lib.dsa_indexer_k_planes_bytes(S) == up(kb * 6144) + up(kb * 4) + up(S * 4)
        for T, H in ((64, 64), (3, 48)):
            full = lib.dsa_indexer_workspace_bytes(T, H, 128, S)
            assert full - lib.dsa_indexer_workspace_bytes_prepared(T, H, 128, S) == \
                lib.dsa_indexer_k_planes_bytes(S)
    assert lib.dsa_indexer_k_planes_bytes(-1) == 0


def _prep_args(**kw):
    a = _lib.KPrepareArgs()
    base = dict(k_idx=0x2000, k_scale=0x3000, num_positions=32768, first_position=0,
                count=32768, k_planes=0x10000, k_planes_capacity=32768)
    base.update(kw)
    for k, v in base.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,needle", [
    (dict(k_planes_capacity=1000), "capacity"),
    (dict(first_position=32000, count=1000), "outside"),
    (dict(count=-1), "negative"),
    (dict(k_planes=0x10010), "256-byte"),
    (dict(k_idx=None), "NULL"),
    (dict(k_idx=0x2004), "aligned"),
    (dict(k_cache=0x9000), "not both"),
    (dict(k_idx=None, k_scale=None, k_cache=0x9000, k_pages=0xa000, k_page_size=6,
          k_num_pages=4), "multiple of 4"),
])
def test_prepare_k_host_validation(kw, needle):
    lib = _lib.load()
    rc = lib.dsa_indexer_prepare_k(ctypes.byref(_prep_args(**kw)), None)
    assert rc == _lib.DSA_EINVAL and needle in lib.dsa_last_error().decode()
    # nothing to prepare: accepted without a launch
    assert lib.dsa_indexer_prepare_k(ctypes.byref(_prep_args(first_position=100, count=0)),
                                     None) == 0


def test_indexer_with_planes_host_validation():
    """Planes laid out for fewer positions than the call reads are refused; a
    call with planes needs no K source and only the smaller workspace."""
    lib = _lib.load()
    small = lib.dsa_indexer_workspace_bytes_prepared(64, 64, 128, 32768)
    a = _idx_args(k_idx=None, k_scale=None, k_planes=0x10000, k_planes_capacity=1000,
                  workspace_bytes=small)
    assert lib.dsa_indexer_topk(ctypes.byref(a), None) == _lib.DSA_EINVAL
    assert b"k_planes" in lib.dsa_last_error()
    a = _idx_args(k_idx=None, k_scale=None, k_planes=0x10000, k_planes_capacity=32768,
                  workspace_bytes=small - 256)
    assert lib.dsa_indexer_topk(ctypes.byref(a), None) == _lib.DSA_EWORKSPACE
    a = _idx_args(k_idx=None, k_scale=None, k_planes=0x10080, k_planes_capacity=32768,
                  workspace_bytes=small)
    assert lib.dsa_indexer_topk(ctypes.byref(a), None) == _lib.DSA_EINVAL


@pytest.mark.parametrize("kw,code,needle", [
    (dict(page_size=6), _lib.DSA_EINVAL, "multiple of 4"),
    (dict(num_tokens=-1), _lib.DSA_EINVAL, "num_tokens"),
    (dict(k=None), _lib.DSA_EINVAL, "NULL"),
    (dict(k=0x1008), _lib.DSA_EINVAL, "aligned"),
    (dict(k_stride=100), _lib.DSA_EINVAL, "aligned"),
    (dict(k_cache=0x3004), _lib.DSA_EINVAL, "aligned"),
])
def test_k_append_host_validation(kw, code, needle):
    lib = _lib.load()
    a = _lib.KAppendArgs()
    base = dict(k=0x1000, k_stride=128, slots=0x2000, num_tokens=16, k_cache=0x3000,
                num_pages=8, page_size=64)
    base.update(kw)
    for k, v in base.items():
        setattr(a, k, v)
    rc = lib.dsa_indexer_k_append(ctypes.byref(a), None)
    assert rc == code and needle in lib.dsa_last_error().decode()
    a.num_tokens = 0
    a.k = 0x1000
    a.k_stride, a.page_size, a.k_cache = 128, 64, 0x3000
    assert lib.dsa_indexer_k_append(ctypes.byref(a), None) == 0   # nothing to do


def test_indexer_accepts_exact_block_table_width():
    """ceil(S / page_size) entries per row suffice (a 1-D table has stride 0)."""
    lib = _lib.load()
    for S, ps, width in ((32768, 64, 512), (1000, 64, 16), (1, 64, 1)):
        a = _idx_args(num_positions=S, block_table=0x7000, page_size=ps, block_table_width=width,
                      num_tokens=0, q_idx=None)
        assert lib.dsa_indexer_topk(ctypes.byref(a), None) == 0
        a = _idx_args(num_positions=S, block_table=0x7000, page_size=ps,
                      block_table_width=width - 1, block_table_stride=0,
                      workspace_bytes=lib.dsa_indexer_workspace_bytes(64, 64, 128, S))
        assert lib.dsa_indexer_topk(ctypes.byref(a), None) == _lib.DSA_EINVAL


def test_reference_argument_lists_raise_type_error_naming_the_layout():
    """The reference's per-sequence entry points (indexer_kernel.py:345-363,
    kernel.py:184-211) take other arguments; calling this build's functions
    with them must say so rather than fail on a shape check."""
    from dsa_amd.indexer_kernel import run_indexer_and_topk, run_sparse_attention_pipeline
    ref_indexer = [None] * 14          # q, k cache, weights, seq_lens, ..., topk
    with pytest.raises(TypeError, match="per-query-token layout"):
        run_indexer_and_topk(*ref_indexer)
    with pytest.raises(TypeError, match="seq_lens"):
        run_indexer_and_topk(None, None, None, None, None, 2048, seq_lens=None)
    with pytest.raises(TypeError, match="per-sequence"):
        run_sparse_attention_pipeline(*([None] * 19))
    with pytest.raises(TypeError, match="batch_size"):
        run_indexer_and_topk(q_index_fp8=None, batch_size=4)
    with pytest.raises(TypeError, match="unexpected keyword"):
        run_indexer_and_topk(None, None, None, None, None, 8, bogus=1)
    with pytest.raises(TypeError, match="missing required"):
        run_indexer_and_topk(None, None, None)
    with pytest.raises(TypeError, match="multiple values"):
        run_indexer_and_topk(None, None, None, None, None, 8, topk=8)


def test_sm_scale_tensor_must_be_one_element():
    from dsa_amd import kernel
    d = workloads.cfg1()
    with pytest.raises(ValueError, match="one-element"):
        kernel(d["q_nope"], d["q_pe"], d["ckv_cache"], d["kpe_cache"], d["sparse_indices"],
               torch.ones(2))
