"""GPU parity of the fused attention prologue (per-head RMSNorm + RoPE in
place, delta_attention/llama.py:60-74, 161-192, qwen3.py:37-43): RoPE is
bit-exact against the reference's own bf16/fp16 torch ops and the oracle's
bf16 restatement; with the norm, every element is within one rounding of the
torch module's (its fp32 mean/rsqrt may round differently in the last bit)."""

import numpy as np
import pytest
import torch

from helpers import np64
from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu


def _proj_views(B, S, Hq, Hkv, D, dtype, seed):
    """q and k as [B,S,H,D] views of one fused projection buffer (token stride
    (Hq + 2 Hkv) D), the layout of a packed qkv GEMM output."""
    g = torch.Generator().manual_seed(seed)
    buf = torch.randn(B, S, (Hq + 2 * Hkv) * D, generator=g).to(dtype).cuda()
    q = buf[..., :Hq * D].view(B, S, Hq, D)
    k = buf[..., Hq * D:(Hq + Hkv) * D].view(B, S, Hkv, D)
    return buf, q, k


def _tables(B, S, D, dtype, per_batch):
    from delta_attention.llama import rope_cos_sin
    pos = torch.arange(S, device="cuda")[None].expand(B, S).contiguous()
    if per_batch:
        pos = pos + torch.arange(B, device="cuda")[:, None] * 37   # distinct offsets per batch
    else:
        pos = pos[:1]
    return rope_cos_sin(pos, D, 500000.0, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [128, 64, 32, 256])
@pytest.mark.parametrize("per_batch", [False, True])
def test_rope_bit_exact(gpu, dtype, D, per_batch):
    from delta_attention import ops
    from delta_attention.llama import apply_rotary_pos_emb
    B, S, Hq, Hkv = 2, 333, 8, 2
    buf, q, k = _proj_views(B, S, Hq, Hkv, D, dtype, seed=D + per_batch)
    cos, sin = _tables(B, S, D, dtype, per_batch)
    ref_q, ref_k = apply_rotary_pos_emb(q.transpose(1, 2).clone(), k.transpose(1, 2).clone(), cos, sin)
    v_before = buf[..., (Hq + Hkv) * D:].clone()
    ops.rope_qk(q, k, cos, sin)
    torch.cuda.synchronize()
    assert torch.equal(q.transpose(1, 2), ref_q) and torch.equal(k.transpose(1, 2), ref_k)
    assert torch.equal(buf[..., (Hq + Hkv) * D:], v_before)     # v untouched


@pytest.mark.parametrize("dtype,D,norm", [(torch.bfloat16, 128, False), (torch.float16, 64, False),
                                          (torch.bfloat16, 32, False), (torch.bfloat16, 256, False),
                                          (torch.bfloat16, 128, True), (torch.float16, 256, True)])
def test_rope_large_inputs(gpu, dtype, D, norm):
    """Inputs of 4 MB and more take the streaming launch (several row pieces
    per thread); an odd token count leaves the last pieces of the grid empty."""
    from delta_attention import ops
    from delta_attention.llama import LlamaRMSNorm, apply_rotary_pos_emb
    B, S, Hq, Hkv = 1, 4099, 32, 8
    assert S * (Hq + Hkv) * D * 2 >= 4 << 20
    buf, q, k = _proj_views(B, S, Hq, Hkv, D, dtype, seed=D + 7)
    cos, sin = _tables(B, S, D, dtype, False)
    v_before = buf[..., (Hq + Hkv) * D:].clone()
    with torch.no_grad():
        if norm:
            qn, kn = LlamaRMSNorm(D, 1e-6).cuda().to(dtype), LlamaRMSNorm(D, 1e-6).cuda().to(dtype)
            torch.nn.init.uniform_(qn.weight, 0.5, 1.5)
            torch.nn.init.uniform_(kn.weight, 0.5, 1.5)
            rq, rk = apply_rotary_pos_emb(qn(q).transpose(1, 2), kn(k).transpose(1, 2), cos, sin)
            ops.rope_qk(q, k, cos, sin, q_norm_w=qn.weight, k_norm_w=kn.weight, eps=1e-6)
        else:
            rq, rk = apply_rotary_pos_emb(q.transpose(1, 2).clone(), k.transpose(1, 2).clone(), cos, sin)
            ops.rope_qk(q, k, cos, sin)
    torch.cuda.synchronize()
    if norm:
        _within_one_rounding(q.transpose(1, 2), rq, "q")
        _within_one_rounding(k.transpose(1, 2), rk, "k")
    else:
        assert torch.equal(q.transpose(1, 2), rq) and torch.equal(k.transpose(1, 2), rk)
    assert torch.equal(buf[..., (Hq + Hkv) * D:], v_before)     # v untouched


@pytest.mark.parametrize("D", [128, 64, 32, 256])
def test_rope_matches_oracle_bf16(gpu, D):
    from delta_attention import ops
    B, S, Hq, Hkv = 1, 200, 4, 1
    _, q, k = _proj_views(B, S, Hq, Hkv, D, torch.bfloat16, seed=5)
    q0 = np64(q).astype(np.float32)
    cos, sin = _tables(B, S, D, torch.bfloat16, False)
    c, s = np64(cos)[0].astype(np.float32), np64(sin)[0].astype(np.float32)
    ops.rope_qk(q, k, cos, sin)
    torch.cuda.synchronize()
    ref = O.apply_rope_bf16(q0, c[None, :, None, :], s[None, :, None, :])
    np.testing.assert_array_equal(np64(q).astype(np.float32), ref)


def _within_one_rounding(got, ref, what):
    g, r = np64(got), np64(ref)
    diff = np.abs(g - r)
    exact = (diff == 0).mean()
    # one bf16 rounding of a normed element moves a RoPE output by at most a few ulps of the row scale
    row_scale = np.abs(r).max(axis=-1, keepdims=True)
    assert (diff <= row_scale * 2.0 ** -6).all(), (what, diff.max())
    assert exact > 0.97, (what, exact)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float16, 128),
                                     (torch.bfloat16, 64), (torch.bfloat16, 32),
                                     (torch.float16, 256)])
def test_rope_with_qk_norm(gpu, dtype, D):
    from delta_attention import ops
    from delta_attention.llama import LlamaRMSNorm, apply_rotary_pos_emb
    B, S, Hq, Hkv = 2, 257, 10, 2
    _, q, k = _proj_views(B, S, Hq, Hkv, D, dtype, seed=9)
    qn, kn = LlamaRMSNorm(D, 1e-6).cuda().to(dtype), LlamaRMSNorm(D, 1e-6).cuda().to(dtype)
    with torch.no_grad():
        torch.nn.init.uniform_(qn.weight, 0.5, 1.5)
        torch.nn.init.uniform_(kn.weight, 0.5, 1.5)
        cos, sin = _tables(B, S, D, dtype, False)
        rq, rk = apply_rotary_pos_emb(qn(q).transpose(1, 2), kn(k).transpose(1, 2), cos, sin)
        ops.rope_qk(q, k, cos, sin, q_norm_w=qn.weight, k_norm_w=kn.weight, eps=1e-6)
    torch.cuda.synchronize()
    _within_one_rounding(q.transpose(1, 2), rq, "q")
    _within_one_rounding(k.transpose(1, 2), rk, "k")


def test_rope_empty_and_k_only(gpu):
    from delta_attention import ops
    from delta_attention.llama import apply_rotary_pos_emb
    _, q, k = _proj_views(1, 0, 4, 1, 128, torch.bfloat16, seed=0)
    cos, sin = _tables(1, 0, 128, torch.bfloat16, False)
    ops.rope_qk(q, k, cos, sin)                 # S = 0: nothing launched
    _, q, k = _proj_views(1, 64, 4, 1, 128, torch.bfloat16, seed=1)
    cos, sin = _tables(1, 64, 128, torch.bfloat16, False)
    q0 = q.clone()
    _, rk = apply_rotary_pos_emb(q.transpose(1, 2).clone(), k.transpose(1, 2).clone(), cos, sin)
    ops.rope_qk(None, k, cos, sin)
    torch.cuda.synchronize()
    assert torch.equal(q, q0) and torch.equal(k.transpose(1, 2), rk)


def test_module_fused_prologue_matches_torch_prologue(gpu):
    """LlamaAttention.forward (fused prologue kernel) against the reference's
    torch prologue (_qkv + apply_rotary_pos_emb) feeding the same delta_forward:
    identical outputs, since the RoPE kernel is bit-exact."""
    import types
    from delta_attention.llama import LlamaAttention, apply_rotary_pos_emb, rope_cos_sin
    cfg = types.SimpleNamespace(
        hidden_size=1024, num_attention_heads=8, num_key_value_heads=2, head_dim=128,
        attention_bias=False, attention_dropout=0.0, rms_norm_eps=1e-6,
        _attn_implementation="window", mode="delta", delta_lambda=64, sliding_window=256,
        sink_tokens=16, stride_policy="fixed", log_drift=False)
    torch.manual_seed(3)
    m = LlamaAttention(cfg, layer_idx=0).cuda().to(torch.bfloat16)
    x = torch.randn(1, 1100, 1024, device="cuda", dtype=torch.bfloat16)
    cos, sin = rope_cos_sin(torch.arange(1100, device="cuda")[None], 128, 500000.0, torch.bfloat16)
    with torch.no_grad():
        y, _ = m(x, (cos, sin))
        q, k, v = m._qkv(x, (1, 1100, -1, 128))
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        a, _ = m.delta_forward(m, q, k, v, None, scaling=m.scaling)
        y_ref = m.o_proj(a.reshape(1, 1100, -1))
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)


@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("D,dtype,pos", [
    (128, torch.bfloat16, 17), (128, torch.bfloat16, 0), (128, torch.bfloat16, 39),
    (64, torch.bfloat16, 39), (64, torch.float16, 0), (128, torch.float16, 39),
    (32, torch.bfloat16, 5), (256, torch.float16, 39),
])
def test_rope_qk_append_equals_rope_then_cache_update(gpu, norm, D, dtype, pos):
    """The one-token decode prologue with the cache append in the same launch:
    q rotated in place and the cache rows at the device-held position hold
    exactly what rope_qk followed by the cache update (index_copy_) writes;
    other cache rows untouched. Positions 0 and L_max - 1 (the last cache row)
    included."""
    from delta_attention import ops
    from delta_attention.llama import rope_cos_sin
    B, Hq, Hkv, L_max = 2, 8, 2, 40
    print(f"rope append B{B} H{Hq}/{Hkv} D{D} {dtype} pos {pos} norm {norm}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(3)
    qkv = torch.randn(B, 1, (Hq + 2 * Hkv) * D, device="cuda", generator=g).to(dtype)
    q = qkv[..., :Hq * D].unflatten(-1, (Hq, D))
    k = qkv[..., Hq * D:(Hq + Hkv) * D].unflatten(-1, (Hkv, D))
    v = qkv[..., (Hq + Hkv) * D:].unflatten(-1, (Hkv, D))
    cos, sin = rope_cos_sin(torch.full((1, 1), pos, device="cuda"), D, 5e5, dtype)
    w = [torch.rand(D, device="cuda", generator=g).to(dtype) + 0.5 for _ in range(2)] if norm else [None, None]
    kc = torch.randn(B, L_max, Hkv, D, device="cuda", generator=g).to(dtype)
    vc = torch.randn(B, L_max, Hkv, D, device="cuda", generator=g).to(dtype)
    kc2, vc2 = kc.clone(), vc.clone()
    q_ref, k_ref = q.clone(), k.clone()
    ops.rope_qk(q_ref, k_ref, cos, sin, q_norm_w=w[0], k_norm_w=w[1], eps=1e-6)
    p = torch.tensor([pos], device="cuda", dtype=torch.int64)
    kc2.index_copy_(1, p, k_ref)
    vc2.index_copy_(1, p, v)
    k_before = k.clone()
    ops.rope_qk_append(q, k, v, cos, sin, kc, vc, p, q_norm_w=w[0], k_norm_w=w[1], eps=1e-6)
    torch.cuda.synchronize()
    assert torch.equal(q, q_ref)
    assert torch.equal(k, k_before)            # k itself is not modified
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)


@pytest.mark.parametrize("pos", [40, -1])
def test_rope_qk_append_position_outside_the_caches(gpu, pos):
    """A device-held position outside [0, max_len) is caught by the kernel's
    own bound: q is rotated as usual, k is kept, and neither cache changes."""
    from delta_attention import ops
    from delta_attention.llama import rope_cos_sin
    B, Hq, Hkv, D, L_max = 1, 8, 2, 128, 40
    print(f"rope append out-of-range pos {pos}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(5)
    q = torch.randn(B, 1, Hq, D, device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn(B, 1, Hkv, D, device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn(B, 1, Hkv, D, device="cuda", generator=g).to(torch.bfloat16)
    cos, sin = rope_cos_sin(torch.full((1, 1), 7, device="cuda"), D, 5e5, torch.bfloat16)
    kc = torch.randn(B, L_max, Hkv, D, device="cuda", generator=g).to(torch.bfloat16)
    vc = torch.randn(B, L_max, Hkv, D, device="cuda", generator=g).to(torch.bfloat16)
    kc0, vc0, k0 = kc.clone(), vc.clone(), k.clone()
    q_ref = q.clone()
    ops.rope_qk(q_ref, None, cos, sin)
    ops.rope_qk_append(q, k, v, cos, sin, kc, vc, torch.tensor([pos], device="cuda"))
    torch.cuda.synchronize()
    assert torch.equal(q, q_ref) and torch.equal(k, k0)
    assert torch.equal(kc, kc0) and torch.equal(vc, vc0)
