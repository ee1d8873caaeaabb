"""GPU parity of the F16 KV cache and GQA decode attention.

Exact path: bit-exact against the oracle's two-pass restatement
(onlineAttentionGroup4F16 model.go:3527-3588).  Split-K path: within
1e-5 relative / 1e-6 absolute of the exact result (configs[3] shapes).
"""
import numpy as np
import pytest

from conftest import normal
from oracle import oracle as ref

pytestmark = pytest.mark.gpu

N_HEADS, N_KV, HD = 32, 8, 128
KVD = N_KV * HD
SCALE = np.float32(1 / np.sqrt(HD))


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def fill_cache(hip, layers, ctx, seed, max_len=None):
    import torch
    kv = hip.KVCacheF16(layers, KVD, KVD, max_len or ctx)
    k = normal(seed, (ctx, KVD))
    v = normal(seed + 1, (ctx, KVD))
    dk, dv = torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
    for pos in range(ctx):
        kv.store_kv_dev(0, pos, dk[pos], dv[pos])
    torch.cuda.synchronize()
    return kv, ref.f32_to_f16(k), ref.f32_to_f16(v)


def test_store_kv_rounds_like_f32_to_f16(hip):
    kv = hip.KVCacheF16(2, KVD, KVD, 16)
    k = normal(1, KVD) * 1000
    v = normal(2, KVD) * 1e-5
    kv.store_kv(1, 5, k, v)
    q = np.zeros(4 * HD, np.float32)
    # attending one position returns exactly that V row (weight 1, denom 1)
    out = kv.attend_head_group(1, 3, q, 4, HD, HD, 5, 5, SCALE)
    vrow = ref.f16_to_f32(ref.f32_to_f16(v))[3 * HD:4 * HD]
    for h in range(4):
        assert np.array_equal(bits(out[h * HD:(h + 1) * HD]), bits(vrow))


@pytest.mark.parametrize("ctx,start", [(1, 0), (7, 0), (513, 0), (640, 0), (300, 123)])
def test_exact_group_attention_bit_exact(hip, ctx, start):
    kv, k16, v16 = fill_cache(hip, 1, ctx, 10 + ctx)
    q = normal(20 + ctx, N_HEADS * HD)
    for g in (0, 5):
        qg = q[g * 4 * HD:(g + 1) * 4 * HD]
        got = kv.attend_head_group(0, g, qg, 4, HD, HD, start, ctx - 1, SCALE)
        want = ref.attend_group_f16(qg, k16.ravel()[g * HD:], v16.ravel()[g * HD:], 4, KVD, KVD,
                                    HD, HD, start, ctx - 1, SCALE)
        assert np.array_equal(bits(got), bits(want)), (ctx, start, g)


def _all_heads_oracle(q, k16, v16, start, end):
    out = np.empty(N_HEADS * HD, np.float32)
    for g in range(N_KV):
        out[g * 4 * HD:(g + 1) * 4 * HD] = ref.attend_group_f16(
            q[g * 4 * HD:(g + 1) * 4 * HD], k16.ravel()[g * HD:], v16.ravel()[g * HD:], 4, KVD,
            KVD, HD, HD, start, end, SCALE)
    return out


def rope_rows(x, first_pos, n_heads, theta=500000.0):
    """Interleaved RoPE (applyPreparedRope, model.go:3051-3093) of row i at
    position first_pos + i, through the oracle's restatement."""
    inv = ref.rope_inv_freq(theta, HD)
    out = np.empty_like(x)
    for i in range(x.shape[0]):
        s, c = ref.rope_sincos(first_pos + i, inv)
        out[i] = ref.rope_apply(x[i], HD, n_heads, s, c)
    return out


@pytest.mark.parametrize("ctx", [4001, 4096, 32768])
def test_decode_attention_configs3(hip, ctx):
    """32 q heads, 8 kv heads, head_dim 128, F16 KV at 4096 and
    32768, RoPE theta 500000 on Q (at the decode position ctx - 1) and on
    every K row (at its own position) before the f16 store.  Exact path
    bit-exact; split-K within 1e-5 relative / 1e-6 absolute."""
    import torch
    kv = hip.KVCacheF16(1, KVD, KVD, ctx)
    k = rope_rows(normal(30, (ctx, KVD)), 0, N_KV)
    v = normal(31, (ctx, KVD))
    dk, dv = torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
    for pos in range(ctx):
        kv.store_kv_dev(0, pos, dk[pos], dv[pos])
    torch.cuda.synchronize()
    k16, v16 = ref.f32_to_f16(k), ref.f32_to_f16(v)
    q = rope_rows(normal(32, (1, N_HEADS * HD)), ctx - 1, N_HEADS)[0]
    dq = torch.from_numpy(q).cuda()
    want = _all_heads_oracle(q, k16, v16, 0, ctx - 1)
    out = torch.empty(N_HEADS * HD, dtype=torch.float32, device="cuda")
    print(f"attention ctx {ctx} exact", flush=True)
    kv.attend_dev(0, dq, N_HEADS, N_KV, HD, 0, ctx - 1, float(SCALE), out, mode=hip.ATTN_EXACT)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out.cpu().numpy()), bits(want))
    print(f"attention ctx {ctx} split-K", flush=True)
    kv.attend_dev(0, dq, N_HEADS, N_KV, HD, 0, ctx - 1, float(SCALE), out, mode=hip.ATTN_SPLITK)
    torch.cuda.synchronize()
    assert np.allclose(out.cpu().numpy(), want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("ctx,start", [(1, 0), (7, 0), (300, 123), (640, 0), (2049, 0),
                                       (3272, 0), (3273, 0)])
def test_decode_attention_whole_span_in_lds(hip, ctx, start):
    """One decode token whose span fits one workgroup's LDS image (the
    one-token values kernel up to 3272 positions, the long-span kernel from
    3273): bit-exact against the oracle for spans that end inside and on the
    32-position value groups and score chunks, and for a window that starts
    past position 0."""
    import torch
    kv, k16, v16 = fill_cache(hip, 1, ctx, 50 + ctx)
    q = normal(51 + ctx, N_HEADS * HD)
    dq = torch.from_numpy(q).cuda()
    out = torch.empty(N_HEADS * HD, dtype=torch.float32, device="cuda")
    print(f"attention whole span ctx {ctx} start {start}", flush=True)
    kv.attend_dev(0, dq, N_HEADS, N_KV, HD, start, ctx - 1, float(SCALE), out, mode=hip.ATTN_EXACT)
    torch.cuda.synchronize()
    want = _all_heads_oracle(q, k16, v16, start, ctx - 1)
    assert np.array_equal(bits(out.cpu().numpy()), bits(want))


def test_splitk_short_spans(hip):
    import torch
    kv, k16, v16 = fill_cache(hip, 1, 200, 40)
    q = normal(41, N_HEADS * HD)
    dq = torch.from_numpy(q).cuda()
    out = torch.empty(N_HEADS * HD, dtype=torch.float32, device="cuda")
    for start, end in ((0, 0), (0, 63), (0, 64), (10, 199), (150, 151)):
        kv.attend_dev(0, dq, N_HEADS, N_KV, HD, start, end, float(SCALE), out, mode=hip.ATTN_SPLITK)
        torch.cuda.synchronize()
        want = _all_heads_oracle(q, k16, v16, start, end)
        assert np.allclose(out.cpu().numpy(), want, rtol=1e-5, atol=1e-6), (start, end)


def test_attention_rejects_bad_ranges(hip):
    kv = hip.KVCacheF16(1, KVD, KVD, 8)
    with pytest.raises(hip.GllmError):
        kv.attend_head_group(0, 0, np.zeros(4 * HD, np.float32), 4, HD, HD, 0, 8, SCALE)
    with pytest.raises(hip.GllmError):
        kv.attend_head_group(0, 0, np.zeros(4 * HD, np.float32), 4, HD, HD, 3, 2, SCALE)
    with pytest.raises(hip.GllmError):
        kv.store_kv(1, 0, np.zeros(KVD, np.float32), np.zeros(KVD, np.float32))
