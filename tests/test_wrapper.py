"""Host semantics of the drop-in wrappers (no GPU): validation errors with the
reference's messages (python/modeling_attention.py:21-147), the mask/score/
attention_mask merge rules, defaults, the HF adapter (modeling_attention.py:150-192),
and that the autograd entry point refuses to run anywhere but on the GPU."""

import pytest
import torch

import tilelang_fa2_4d_mask as api
from tilelang_fa2_4d_mask import modeling_attention as MA


class Recorder:
    def __init__(self):
        self.calls = []

    def __call__(self, *args):
        self.calls.append(args)
        q = args[0]
        return torch.zeros_like(q)


@pytest.fixture
def rec(monkeypatch):
    r = Recorder()
    monkeypatch.setattr(MA, "flash_attention_with_4d_mask", r)
    return r


def qkv(B=2, Hq=4, Hk=2, Tq=5, Tk=7, D=8, layout="bhsd", dtype=torch.bfloat16):
    if layout == "bhsd":
        return (torch.randn(B, Hq, Tq, D).to(dtype), torch.randn(B, Hk, Tk, D).to(dtype),
                torch.randn(B, Hk, Tk, D).to(dtype))
    return (torch.randn(B, Tq, Hq, D).to(dtype), torch.randn(B, Tk, Hk, D).to(dtype),
            torch.randn(B, Tk, Hk, D).to(dtype))


def test_positional_contract_and_defaults(rec):
    q, k, v = qkv()
    api.tilelang_flash_attention(q, k, v)
    (Q, K, V, mask, score, scale, causal, atomic, bhsd) = rec.calls[-1]
    assert Q is q and K is k and V is v and mask is None and score is None
    assert scale == pytest.approx(8 ** -0.5) and causal is False and atomic is True and bhsd is True
    qs, ks, vs = qkv(layout="bshd")
    api.tilelang_flash_attention(qs, ks, vs, layout="bshd", is_causal=True, scale=0.25, use_atomic_backward=False)
    (_, _, _, _, _, scale, causal, atomic, bhsd) = rec.calls[-1]
    assert scale == 0.25 and causal is True and atomic is False and bhsd is False


@pytest.mark.parametrize(
    "mutate,msg",
    [
        (lambda q, k, v: (q[0], k, v), "query, key, and value must be rank-4 tensors"),
        (lambda q, k, v: (q, k[:1], v), "query, key, and value must have the same batch size"),
        (lambda q, k, v: (q, k, v[:, :, :3]), "key and value must have the same sequence length"),
        (lambda q, k, v: (q, k, v[:, :1]), "key and value must have the same number of heads"),
        (lambda q, k, v: (q, k[..., :4], v[..., :4]), "query, key, and value must have the same head dimension"),
        (lambda q, k, v: (q[:, :3], k, v), "query heads (3) must be divisible by key/value heads (2)"),
        (lambda q, k, v: (q.float(), k.float(), v.float()), "TileLang attention expects fp16 or bf16 inputs"),
        (lambda q, k, v: (q, k.half(), v), "query, key, and value must have the same dtype"),
    ],
)
def test_validation_messages(rec, mutate, msg):
    q, k, v = mutate(*qkv())
    with pytest.raises(ValueError) as e:
        api.tilelang_flash_attention(q, k, v)
    assert msg in str(e.value)


def test_layout_error(rec):
    q, k, v = qkv()
    with pytest.raises(ValueError, match="unsupported layout: bsdh"):
        api.tilelang_flash_attention(q, k, v, layout="bsdh")


def test_mask_and_score_validation(rec):
    q, k, v = qkv()
    with pytest.raises(ValueError, match="mask must be a bool tensor with True for valid entries"):
        api.tilelang_flash_attention(q, k, v, mask=torch.ones(2, 4, 5, 7))
    with pytest.raises(ValueError, match=r"mask must have shape \[B, H or 1, Tq, Tk\]"):
        api.tilelang_flash_attention(q, k, v, mask=torch.ones(4, 5, 7, dtype=torch.bool))
    with pytest.raises(ValueError, match=r"mask has trailing shape \(5, 6\), expected \(5, 7\)"):
        api.tilelang_flash_attention(q, k, v, mask=torch.ones(2, 4, 5, 6, dtype=torch.bool))
    with pytest.raises(ValueError, match="mask batch dimension must be 1 or 2"):
        api.tilelang_flash_attention(q, k, v, mask=torch.ones(3, 4, 5, 7, dtype=torch.bool))
    with pytest.raises(ValueError, match="mask head dimension must be 1 or 4"):
        api.tilelang_flash_attention(q, k, v, mask=torch.ones(2, 2, 5, 7, dtype=torch.bool))
    with pytest.raises(ValueError, match="score must be a floating-point tensor"):
        api.tilelang_flash_attention(q, k, v, score=torch.ones(2, 4, 5, 7, dtype=torch.int32))
    with pytest.raises(ValueError, match="attention_mask must be bool or floating point"):
        api.tilelang_flash_attention(q, k, v, attention_mask=torch.ones(2, 4, 5, 7, dtype=torch.int64))


def test_broadcast_masks_are_views_not_copies(rec):
    q, k, v = qkv()
    m = torch.rand(1, 1, 5, 7) > 0.3
    api.tilelang_flash_attention(q, k, v, mask=m)
    mask = rec.calls[-1][3]
    assert mask.shape == (2, 4, 5, 7) and mask.stride()[:2] == (0, 0)
    assert mask.data_ptr() == m.data_ptr()
    assert torch.equal(mask, m.expand(2, 4, 5, 7))


def test_merge_rules(rec):
    q, k, v = qkv()
    m = torch.rand(2, 4, 5, 7) > 0.3
    am_bool = torch.rand(2, 1, 5, 7) > 0.2
    api.tilelang_flash_attention(q, k, v, mask=m, attention_mask=am_bool)
    assert torch.equal(rec.calls[-1][3], m & am_bool.expand(2, 4, 5, 7))
    s = torch.randn(1, 4, 5, 7, dtype=torch.float16)
    am = torch.randn(2, 4, 5, 7)
    api.tilelang_flash_attention(q, k, v, score=s, attention_mask=am, scale=0.5)
    score = rec.calls[-1][4]
    assert score.dtype == torch.float32
    assert torch.allclose(score, s.float().expand(2, 4, 5, 7) + am / 0.5)
    api.tilelang_flash_attention(q, k, v, attention_mask=am, scale=0.5, attention_mask_is_scaled=False)
    assert torch.allclose(rec.calls[-1][4], am)


def test_hf_adapter(rec):
    q, k, v = qkv()

    class M:
        is_causal = True

    class N:
        is_causal = False

    out, w = api.tilelang_attention_forward(M(), q, k, v, None, 0.3)
    assert w is None and rec.calls[-1][6] is True and rec.calls[-1][5] == 0.3
    api.tilelang_attention_forward(N(), q, k, v, None, 0.3)
    assert rec.calls[-1][6] is False
    api.tilelang_attention_forward(object(), q, k, v, None, 0.3)  # no attribute: causal
    assert rec.calls[-1][6] is True
    am = torch.zeros(2, 1, 5, 7)
    api.tilelang_attention_forward(M(), q, k, v, am, 0.3)
    assert rec.calls[-1][6] is False
    api.tilelang_attention_forward(M(), q, k, v, am, 0.3, is_causal=True, use_atomic_backward=False)
    assert rec.calls[-1][6] is True and rec.calls[-1][7] is False
    with pytest.raises(ValueError, match="TileLang FA2 wrapper does not implement attention dropout"):
        api.tilelang_attention_forward(M(), q, k, v, None, 0.3, dropout=0.1)
    api.tilelang_attention_forward(M(), q, k, v, None, 0.3, dropout=None)


def test_function_refuses_cpu_tensors():
    q, k, v = qkv()
    with pytest.raises(ValueError, match="runs on the GPU"):
        api.flash_attention_with_4d_mask(q, k, v, None, None, None, False, True, True)
    with pytest.raises(AssertionError):
        api.flash_attention_with_4d_mask(q[0], k, v, None, None, None, False, True, True)


def test_kernel_head_dim_padding_rule():
    """Head dims the kernels are built for run as they are; others up to 256 run
    at the next built one (zero-padded, exact); larger ones are passed through for
    the library to reject."""
    from tilelang_fa2_4d_mask import fa2

    assert fa2.KERNEL_HEAD_DIMS == (64, 128, 256)
    assert [fa2.kernel_head_dim(d) for d in (8, 32, 63, 64, 65, 96, 112, 128)] == [64, 64, 64, 64, 128, 128, 128, 128]
    assert [fa2.kernel_head_dim(d) for d in (129, 160, 192, 255, 256)] == [256] * 5
    assert fa2.kernel_head_dim(257) == 257 and fa2.kernel_head_dim(512) == 512
    x = torch.randn(2, 3, 4, 96)
    y = fa2._pad_head_dim(x, 128)
    assert y.shape == (2, 3, 4, 128) and torch.equal(y[..., :96], x) and not y[..., 96:].any()
    assert fa2._pad_head_dim(x, 96) is x


def test_long_rows_are_relaid_head_major():
    """The backward reaches a Q / dO row with a 32-bit byte offset from its
    head's first row: (Tq + 32) rows spanning 4 GiB or more (token-major, 32
    heads of 128 at 540k tokens) are re-laid head-major, shorter ones pass
    through as the same tensor (meta tensors: no memory)."""
    from tilelang_fa2_4d_mask import fa2

    big = torch.empty((1, 540000, 32, 128), dtype=torch.bfloat16, device="meta")
    assert (540000 + 32) * 2 * big.stride(1) >= fa2.ROW_SPAN_LIMIT
    out = fa2._rows_reachable(big, 540000)
    assert out.shape == big.shape
    assert out.stride() == (32 * 540000 * 128, 128, 540000 * 128, 1)
    assert (540000 + 32) * 2 * out.stride(1) < fa2.ROW_SPAN_LIMIT
    small = torch.empty((1, 500000, 32, 128), dtype=torch.bfloat16, device="meta")
    assert fa2._rows_reachable(small, 500000) is small
    # a head-major view of token-major storage is left as it is
    hm = big.transpose(1, 2).contiguous().transpose(1, 2)
    assert fa2._rows_reachable(hm, 540000) is hm
