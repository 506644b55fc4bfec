"""The torch.library operators without a GPU: their schemas, their fake
implementations (shapes and dtypes under FakeTensorMode, as torch.compile
traces them) and the dispatcher's refusal of CPU tensors (no CPU fallback)."""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from bmx_amd import k2b, ops, rtn


def test_operators_registered_with_their_schemas():
    for name in ("k2b_decode", "k2b_append", "rtn_decode", "rtn_append", "prefill_attention"):
        op = getattr(torch.ops.bmx, name).default
        assert op._schema.name == f"bmx::{name}"
    for name in ("k2b_append", "rtn_append"):   # the page pool is the one argument written
        sch = getattr(torch.ops.bmx, name).default._schema
        assert [a.name for a in sch.arguments if a.alias_info is not None and a.alias_info.is_write] == ["pages"]
    for name in ("k2b_decode", "rtn_decode", "prefill_attention"):   # fresh outputs only
        sch = getattr(torch.ops.bmx, name).default._schema
        assert all(a.alias_info is None for a in sch.arguments)


@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
def test_fake_decode_gives_the_query_shape_and_dtype(dt):
    c = k2b.CodecConsts.make()
    with FakeTensorMode():
        q = torch.empty(2, 8, 4, 128, dtype=dt, device="cuda")
        pages = torch.empty(256, k2b.page_bytes(8, 32), dtype=torch.uint8, device="cuda")
        table = torch.empty(2, 64, dtype=torch.int32, device="cuda")
        ln = torch.empty(2, dtype=torch.int32, device="cuda")
        basis = torch.empty(1024, 32, dtype=torch.float16, device="cuda")
        o = torch.ops.bmx.k2b_decode(q, pages, table, ln, 1024, basis, sm_scale=128 ** -0.5, rank=32,
                                     **ops.consts_args(c))
        assert o.shape == q.shape and o.dtype == dt and o.device.type == "cuda"
        rp = torch.empty(256, rtn.page_bytes(8, k_bits=4, v_bits=4, k_group=32, v_group=32),
                         dtype=torch.uint8, device="cuda")
        o = torch.ops.bmx.rtn_decode(q, rp, table, ln, 1024, 128 ** -0.5, 4, 4, 32, 32)
        assert o.shape == q.shape and o.dtype == dt


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_fake_prefill_gives_the_query_shape_and_dtype(dt):
    with FakeTensorMode():
        q = torch.empty(16, 100, 128, dtype=dt, device="cuda").transpose(0, 1).transpose(0, 1)
        k = torch.empty(4, 900, 128, dtype=dt, device="cuda")
        o = torch.ops.bmx.prefill_attention(q, k, k, 128 ** -0.5, True)
        assert o.shape == (16, 100, 128) and o.dtype == dt and o.is_contiguous()


def test_cpu_tensors_are_refused_by_the_dispatcher():
    c = k2b.CodecConsts.make()
    with pytest.raises(NotImplementedError, match="CPU"):
        torch.ops.bmx.k2b_decode(torch.zeros(1, 8, 4, 128), torch.zeros(64, k2b.page_bytes(8, 32), dtype=torch.uint8),
                                 None, torch.zeros(1, dtype=torch.int32), 1024,
                                 torch.zeros(1024, 32, dtype=torch.float16), sm_scale=0.1, rank=32,
                                 **ops.consts_args(c))
