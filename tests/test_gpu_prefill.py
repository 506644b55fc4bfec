"""bmx_prefill (the MFMA flash attention of the packed cache's prefill) against
attention computed in fp32 on the device, over the masks a cached prefill
carries (chunked_attention.py:320-395 hands them to SDPA): the causal mask of
the last n_q positions (bottom-right aligned, test_packed_streaming.py:122-153
builds it for the two-block prefill), the square causal mask and none.

Tolerances: fp16 atol = rtol = 2e-3 (P and the output rounded to fp16, each a
relative 2^-11), bf16 atol = rtol = 1.6e-2 (2^-8)."""
import pytest
import torch

from bmx_amd import prefill

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL = {torch.float16: (2e-3, 2e-3), torch.bfloat16: (1.6e-2, 1.6e-2)}


def _ref(q, k, v, scale, causal):
    """fp32 attention, the G query heads of a kv head as one batch of rows."""
    hq, n_q, d = q.shape
    h_kv, n_kv, _ = k.shape
    G = hq // h_kv
    qf = q.float().reshape(h_kv, G * n_q, d)
    s = torch.matmul(qf, k.float().transpose(1, 2).contiguous()) * scale
    if causal:
        i = torch.arange(n_q, device=q.device).repeat(G)
        j = torch.arange(n_kv, device=q.device)
        s = s.masked_fill(j[None, None, :] > i[None, :, None] + (n_kv - n_q), float("-inf"))
    return torch.matmul(torch.softmax(s, -1), v.float().contiguous()).reshape(hq, n_q, d)


def _inputs(h_kv, G, n_q, n_kv, dtype, seed, kscale=1.0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(h_kv * G, n_q, 128, device=DEV, generator=g).to(dtype)
    k = (kscale * torch.randn(h_kv, n_kv, 128, device=DEV, generator=g)).to(dtype)
    v = torch.randn(h_kv, n_kv, 128, device=DEV, generator=g).to(dtype)
    return q, k, v


CASES = [
    # h_kv, G, n_q, n_kv, causal, n_split
    (8, 4, 512, 8704, True, 0),      # the bench's 8k cached prefill (auto splits)
    (8, 4, 512, 8704, True, 1),
    (2, 4, 100, 1000, True, 3),      # ragged row tile and key tile
    (1, 1, 64, 64, True, 0),         # square causal
    (2, 8, 130, 130, True, 2),
    (3, 2, 77, 300, False, 0),       # no mask
    (2, 4, 1, 37, True, 0),          # one query
    (2, 4, 5, 5000, True, 16),
    (1, 4, 3, 70, True, 16),         # most splits empty (2 key tiles)
    (1, 3, 50, 129, True, 5),        # G = 3: row tiles span heads unevenly
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("case", CASES)
def test_prefill_matches_fp32_attention(case, dtype):
    h_kv, G, n_q, n_kv, causal, n_split = case
    print(f"prefill case {case} {dtype}", flush=True)
    q, k, v = _inputs(h_kv, G, n_q, n_kv, dtype, seed=n_q * 7 + n_kv)
    scale = 128 ** -0.5
    out = prefill.attention(q, k, v, scale, causal=causal, n_split=n_split)
    torch.cuda.synchronize()
    atol, rtol = TOL[dtype]
    torch.testing.assert_close(out.float(), _ref(q, k, v, scale, causal), atol=atol, rtol=rtol)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_strided_operands_and_peaked_scores(dtype):
    """q as the model hands it over (a transposed view of (n_q, Hq, 128)),
    K/V rows inside a longer buffer, and keys scaled so that the softmax is
    dominated by a few keys per row."""
    h_kv, G, n_q, n_kv = 4, 4, 200, 1500
    print(f"prefill strided {dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(11)
    qb = torch.randn(n_q, h_kv * G, 128, device=DEV, generator=g).to(dtype)
    q = qb.transpose(0, 1)
    kb = (6.0 * torch.randn(h_kv, n_kv + 40, 128, device=DEV, generator=g)).to(dtype)
    vb = torch.randn(h_kv, n_kv + 40, 128, device=DEV, generator=g).to(dtype)
    k, v = kb[:, :n_kv], vb[:, :n_kv]
    scale = 128 ** -0.5
    out = prefill.attention(q, k, v, scale, causal=True)
    torch.cuda.synchronize()
    atol, rtol = TOL[dtype]
    torch.testing.assert_close(out.float(), _ref(q, k, v, scale, True), atol=atol, rtol=rtol)


def test_prefill_splits_agree():
    """The split count changes only the summation order: every split count
    gives the one-split result to fp16 rounding."""
    q, k, v = _inputs(2, 4, 256, 4096, torch.float16, seed=5)
    base = prefill.attention(q, k, v, 0.09, causal=True, n_split=1).float()
    for s in (2, 7, 16):
        out = prefill.attention(q, k, v, 0.09, causal=True, n_split=s).float()
        torch.testing.assert_close(out, base, atol=1e-3, rtol=1e-3)


def test_prefill_rejects_bad_operands():
    q, k, v = _inputs(1, 4, 8, 16, torch.float16, seed=1)
    with pytest.raises(ValueError):
        prefill.attention(q, k[..., :64], v[..., :64], 0.1, causal=True)
    with pytest.raises(RuntimeError, match="n_q <= n_kv"):
        prefill.attention(torch.cat([q, q, q], 1), k, v, 0.1, causal=True)
