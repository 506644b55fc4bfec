"""CPU stand-in for the three kernels under the product cache's host logic
(test infrastructure only).

``OracleLayer`` subclasses bmx_amd.cache.PackedStreamingLayer and keeps its
``update`` -- flush schedule, pre-RoPE stash and slab pruning, blended
bits-per-entry -- while the encode, decode and prefill steps run the CPU oracle
(the reference's codec and attention restated, oracle/): codes per committed
codec page, keys dequantized and rotated with fp16-cast RoPE tables
(packed_streaming.py:79-113, chunked_attention.py:148-189), one softmax over
committed + recent tokens.  ``v_fp16`` encodes values from their fp16 rounding,
as the product's write kernel does."""

from __future__ import annotations

import torch
import torch.nn.functional as F

from bmx_amd import cache as product
from oracle import attention as A
from oracle import codecs as OC
from oracle import spectral as OS


class SpectralOracleStore:
    """Committed spectral codec pages on the CPU: codes by oracle/spectral
    (fixed-order encode, MSE-refined RTN, fp16 steps as stored), keys
    dequantized pre-RoPE, values by the per-head value codec."""

    def __init__(self, pack, h_kv, v_seed, v_fp16, payload="rtn", v_full=False):
        self.pack, self.h_kv, self.v_seed, self.v_fp16 = pack, h_kv, v_seed, v_fp16
        self.v_h = 1 if v_full else h_kv   # full-C turboquant_mse: the per-head codec at h = 1
        self.L = OS.Layout(pack.bits.numpy())
        self.lloyd = ({b: OC.gaussian_codebook(b).numpy() for b in set(self.L.slice_bits.tolist())}
                      if payload == "lloyd" else None)
        self.k, self.v = [], []

    def commit(self, k_pre, v):
        M = OC.to_matrix(k_pre.float().cpu()).numpy()
        codes, scales = OS.quantize(OS.encode(M, self.pack.enc.numpy(), self.L), self.L, self.lloyd)
        K = OS.dequant(codes, scales, self.pack.dec.numpy(), self.L, lloyd=self.lloyd)
        self.k.append(OC.from_matrix(torch.from_numpy(K).float(), self.h_kv))
        vp = v.half().float() if self.v_fp16 else v.float()
        idx, norms, _ = OC.quantize_v_perhead(OC.to_matrix(vp.cpu()), bits=2, seed=self.v_seed, h=self.v_h)
        self.v.append(OC.from_matrix(OC.dequant_v_perhead(idx, norms, bits=2, seed=self.v_seed,
                                                          h=self.v_h), self.h_kv))

    def dense_k_pre(self):
        return torch.cat(self.k, dim=1)

    def dense_v(self):
        return torch.cat(self.v, dim=1)


class OracleLayer(product.PackedStreamingLayer):
    v_fp16 = False

    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        if self._path == "spectral":
            self._oc = SpectralOracleStore(self._pack, self._h_kv, self.v_spec.seed, self.v_fp16,
                                           self.k_spec.payload_quant, self.v_spec.arm == "turboquant_mse")
        else:
            self._oc = A.K2bOracleCache(self._h_kv, self._d_head, self._rank, group=self.k_spec.group,
                                        k_bits=self.k_spec.bits, v_seed=self.v_spec.seed)

    def _commit_spectral(self, k_pre, v):
        self._oc.v_fp16 = self.v_fp16
        self._oc.commit(k_pre, v)

    def _commit(self, k_pre, v):
        for p in range(k_pre.shape[1] // product.PAGE):
            sl = slice(p * product.PAGE, (p + 1) * product.PAGE)
            vp = v[:, sl].half().float() if self.v_fp16 else v[:, sl].float()
            self._oc.commit(k_pre[:, sl].cpu(), vp.cpu())

    def _kv(self, dtype):
        P = self._committed_S_q
        ks, vs = [], []
        if P:
            memo = getattr(self, "_kv_memo", None)   # the committed part changes only at a commit
            if memo is None or memo[0] != (P, dtype):
                cos, sin = product._rope_tables(self._inv_freq, self._rope_scaling, 0, P, "cpu")
                kc = A.apply_rope(self._oc.dense_k_pre(), cos.float(), sin.float()).to(dtype)
                memo = self._kv_memo = ((P, dtype), kc, self._oc.dense_v().to(dtype))
            ks.append(memo[1])
            vs.append(memo[2])
        kw, vw = self.window()   # the product layer's window (its newest row stored)
        if kw is not None and kw.shape[2]:
            ks.append(kw.squeeze(0).cpu().to(dtype))
            vs.append(vw.squeeze(0).cpu().to(dtype))
        return torch.cat(ks, dim=1), torch.cat(vs, dim=1)

    def attend(self, q, scaling, is_causal=False, attention_mask=None):
        if q.device.type != "cpu":   # model on a GPU: the oracle attends on the host
            out = self.attend(q.cpu(), scaling, is_causal, None if attention_mask is None else attention_mask.cpu())
            return out.to(q.device)
        n_heads, n_q, d = q.shape
        G = n_heads // self._h_kv
        Kd, Vd = self._kv(q.dtype)   # rounded to the model dtype, as the product's are
        if n_q == 1 and not is_causal:
            return A.grouped_dense_attention(q.float(), Kd, Vd, G, scaling).to(q.dtype)
        Kx, Vx = Kd.float().repeat_interleave(G, dim=0), Vd.float().repeat_interleave(G, dim=0)
        causal = is_causal and n_q > 1
        return F.scaled_dot_product_attention(
            q.float().unsqueeze(0), Kx.unsqueeze(0), Vx.unsqueeze(0), attn_mask=attention_mask,
            is_causal=causal and attention_mask is None, scale=scaling).squeeze(0).to(q.dtype)


class OracleCache(product.PackedStreamingCache):
    def __init__(self, *args, v_fp16=False, **kwargs):
        super().__init__(*args, **kwargs)

        def _make_layer():
            pack = self._packs.get(len(self.layers)) if self._packs else None
            lay = OracleLayer(self.k_spec, self.v_spec, self.model_config, self.recent_window, pack=pack)
            lay.v_fp16 = v_fp16
            return lay

        self._make_layer = _make_layer
