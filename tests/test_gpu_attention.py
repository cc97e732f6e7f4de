"""Attention consumer on the GPU: decode attention over gathered bf16 K / V
(flash_attn_with_kvcache call shape of
sglang/srt/layers/attention/v1_native/backend.py:306-315) against the
float64 oracle and a plain torch float32 reference.  Tolerance (bf16 output):
|out - ref| <= 1e-2 + 1e-2 * |ref|."""
import importlib
import math
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
from oracle import v1 as O  # noqa: E402

pytestmark = pytest.mark.gpu

AT = importlib.import_module("10_20_amd.attention")
NK = importlib.import_module("10_20_amd.native_kernels")
DEV = "cuda:0"


def _close(got, ref):
    return np.abs(got - ref) <= 1e-2 + 1e-2 * np.abs(ref)


def _torch_ref(q, k, v, scale, lens):
    """softmax(scale q k^T) v in float32 on the GPU, one row at a time."""
    B, _, Hq, D = q.shape
    G = Hq // k.shape[2]
    out = torch.zeros((B, Hq, D), device=DEV)
    for b in range(B):
        n = int(lens[b]) if lens is not None else k.shape[1]
        if n == 0:
            continue
        kk = k[b, :n].float().permute(1, 0, 2).contiguous()   # [Hkv, n, D]
        vv = v[b, :n].float().permute(1, 0, 2).contiguous()
        qq = q[b, 0].float().reshape(k.shape[2], G, D)          # [Hkv, G, D]
        s = torch.matmul(qq, kk.transpose(1, 2).contiguous()) * scale
        out[b] = torch.matmul(torch.softmax(s, -1), vv).reshape(Hq, D)
    return out.cpu().numpy()


@pytest.mark.parametrize("B,S,Hq,Hkv,lens", [(64, 2048, 4, 1, None), (33, 1000, 8, 2, "random"),
                                             (16, 2048, 2, 2, "edges"), (8, 12288 // 4, 4, 1, None)])
def test_decode_attention_vs_oracle(B, S, Hq, Hkv, lens):
    print("attention", B, S, Hq, Hkv, lens, flush=True)
    g = torch.Generator(device=DEV).manual_seed(B * S + Hq)
    q = torch.randn((B, 1, Hq, 128), device=DEV, generator=g).to(torch.bfloat16)
    k = torch.randn((B, S, Hkv, 128), device=DEV, generator=g).to(torch.bfloat16)
    v = torch.randn((B, S, Hkv, 128), device=DEV, generator=g).to(torch.bfloat16)
    seqlens = None
    if lens == "random":
        seqlens = torch.randint(0, S + 1, (B,), device=DEV, generator=g, dtype=torch.int32)
    elif lens == "edges":
        seqlens = torch.tensor([0, 1, 2, 15, 16, 17, 63, 64, 65, 1023, 2047, 2048, 5000, -3, 700, 1],
                               device=DEV, dtype=torch.int32)
    scale = 1.0 / math.sqrt(128)
    out = AT.flash_attn_with_kvcache(q, k, v, cache_seqlens=seqlens, softmax_scale=scale, causal=False)
    got = out[:, 0].float().cpu().numpy()
    ln = None if seqlens is None else np.clip(seqlens.cpu().numpy(), 0, S)
    ref = O.decode_attention(q[:, 0].float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                             scale, ln)
    assert _close(got, ref).all(), float(np.abs(got - ref).max())
    tref = _torch_ref(q, k, v, scale, ln)
    assert _close(got, tref).all()
    if ln is not None:
        assert (got[ln == 0] == 0).all()


def test_consumer_after_gather_workspace():
    # backend.py:300-315: GatherWorkspace.gather -> flash_attn_with_kvcache(qs[:, None], kg, vg)
    g = torch.Generator(device=DEV).manual_seed(5)
    slots, rows = 50000, 128
    kp = torch.randn((slots, 2, 128), device=DEV, generator=g).to(torch.bfloat16)
    vp = torch.randn((slots, 2, 128), device=DEV, generator=g).to(torch.bfloat16)
    req = torch.randperm(slots, device=DEV, generator=g).to(torch.int32)
    ids = torch.randint(0, slots, (rows, 2048), device=DEV, generator=g, dtype=torch.int32)
    q3 = torch.randn((rows, 8, 128), device=DEV, generator=g).to(torch.bfloat16)
    work = NK.GatherWorkspace(rows, DEV, torch.bfloat16)
    for head in (0, 1):
        kg, vg = work.gather(kp, vp, req, ids, head)
        qs = q3[:, head * 4:(head + 1) * 4].contiguous()
        out = AT.flash_attn_with_kvcache(qs[:, None], kg, vg, causal=False, softmax_scale=0.0883883)
        got = out[:, 0].float().cpu().numpy()
        ref = O.decode_attention(qs.float().cpu().numpy(), kg.float().cpu().numpy(), vg.float().cpu().numpy(),
                                 0.0883883)
        assert _close(got, ref).all()
        # the workspace holds exactly the slots' rows of this head
        sel = req[ids.long()].long()
        assert torch.equal(kg[:, :, 0], kp[sel, head]) and torch.equal(vg[:, :, 0], vp[sel, head])


def test_rejects_unsupported_shapes():
    q = torch.zeros((2, 1, 8, 128), device=DEV, dtype=torch.bfloat16)
    kv = torch.zeros((2, 16, 1, 128), device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        AT.flash_attn_with_kvcache(q, kv, kv)  # 8 query heads per KV head
    with pytest.raises(ValueError):
        AT.flash_attn_with_kvcache(q[:, :, :4].float(), kv, kv)
    with pytest.raises(NotImplementedError):
        AT.flash_attn_with_kvcache(q[:, :, :4], kv, kv, k=kv)


@pytest.mark.parametrize("heads", [4, 1])
def test_attend_slots_equals_gather_then_attention(heads):
    # the fused form reads the pools through the slot map: bit-identical to gather + attention,
    # including ids below zero or past the map and map entries outside the pool (zero keys)
    g = torch.Generator(device=DEV).manual_seed(11 + heads)
    slots, rows = 30000, 96
    kp = torch.randn((slots, 2, 128), device=DEV, generator=g).to(torch.bfloat16)
    vp = torch.randn((slots, 2, 128), device=DEV, generator=g).to(torch.bfloat16)
    req = torch.randperm(slots, device=DEV, generator=g).to(torch.int32)
    req[:50] = slots + 7        # past the pool
    req[50:60] = -2             # negative map entries
    ids = torch.randint(-5, slots + 100, (rows, 2048), device=DEV, generator=g, dtype=torch.int32)
    qs = torch.randn((rows, heads, 128), device=DEV, generator=g).to(torch.bfloat16)
    work = NK.GatherWorkspace(rows, DEV, torch.bfloat16)
    for head in (0, 1):
        kg, vg = work.gather(kp, vp, req, ids, head)
        two = AT.flash_attn_with_kvcache(qs[:, None], kg, vg, causal=False, softmax_scale=0.09)
        one = AT.attend_slots(qs, kp, vp, req, ids, head, softmax_scale=0.09)
        assert torch.equal(one, two)
