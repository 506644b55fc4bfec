"""The dense fp16 decode kernel bench.py's comparator runs (bmx_fp16_decode,
include/bmx_bench.h) against a plain fp32 PyTorch attention of the same
step: every query group size it takes, token counts that leave a partial
last chunk, more splits than chunks and token streams with no token at all
(5 tokens), strided head layouts."""
import ctypes as ct

import pytest
import torch

from bmx_amd import _lib

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _run(q, K, V, n_split, sm_scale):
    h, G, D = q.shape
    T = K.shape[1]
    out = torch.empty(h, G, D, dtype=torch.float16, device=DEV)
    ws = torch.empty(int(_lib.lib().bmx_fp16_decode_workspace_bytes(h, G, n_split)), dtype=torch.uint8, device=DEV)
    a = _lib.Fp16DecodeArgs()
    a.q, a.k, a.v = q.data_ptr(), K.data_ptr(), V.data_ptr()
    a.stride_h, a.stride_t = K.stride(0), K.stride(1)
    a.h_kv, a.n_q_groups, a.T, a.n_split = h, G, T, n_split
    a.sm_scale = sm_scale
    a.out, a.workspace, a.workspace_bytes = out.data_ptr(), ws.data_ptr(), ws.numel()
    rc = _lib.lib().bmx_fp16_decode(ct.byref(a), torch.cuda.current_stream(DEV).cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    return out


def _ref(q, K, V, sm_scale):
    s = torch.einsum("hgd,htd->hgt", q.float().cpu(), K.float().cpu()) * sm_scale
    return torch.einsum("hgt,htd->hgd", torch.softmax(s, dim=-1), V.float().cpu())


@pytest.mark.parametrize("G", [1, 2, 4, 8])
@pytest.mark.parametrize("T,n_split", [(1000, 7), (4096, 16), (333, 12), (5, 1), (37, 3)])
def test_fp16_decode_matches_fp32_attention(G, T, n_split):
    gen = torch.Generator(device=DEV).manual_seed(T + G)
    h, D = 8, 128
    q = torch.randn(h, G, D, generator=gen, device=DEV).half()
    K = (2.0 * torch.randn(h, T, D, generator=gen, device=DEV)).half()
    V = torch.randn(h, T, D, generator=gen, device=DEV).half()
    out = _run(q, K, V, n_split, D ** -0.5)
    ref = _ref(q, K, V, D ** -0.5)
    err = (out.float().cpu() - ref).abs().max().item()
    print(f"G {G} T {T} splits {n_split}: max_abs {err:.2e}", flush=True)
    assert err < 4e-3


def test_fp16_decode_strided_heads():
    """Heads at a stride larger than T rows (a cache with room to grow)."""
    gen = torch.Generator(device=DEV).manual_seed(3)
    h, G, D, T, cap = 8, 4, 128, 700, 1024
    q = torch.randn(h, G, D, generator=gen, device=DEV).half()
    Kb = torch.randn(h, cap, D, generator=gen, device=DEV).half()
    Vb = torch.randn(h, cap, D, generator=gen, device=DEV).half()
    out = _run(q, Kb[:, :T], Vb[:, :T], 5, 0.1)
    ref = _ref(q, Kb[:, :T], Vb[:, :T], 0.1)
    assert (out.float().cpu() - ref).abs().max().item() < 4e-3


def test_fp16_decode_rejects_bad_arguments():
    a = _lib.Fp16DecodeArgs()
    assert _lib.lib().bmx_fp16_decode(ct.byref(a), None) != 0   # null pointers
