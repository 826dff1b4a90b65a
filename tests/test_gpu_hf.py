"""The real caller: ``tilelang_attention_forward`` (python/modeling_attention.py:150-192)
as the attention function of a HuggingFace Llama model (README.md:57-77).

A tiny LlamaModel (4 query heads, 2 kv heads, head_dim 64, 2 layers) runs in bf16 on
the GPU with the adapter registered as a transformers attention interface.  Two
registrations cover both mask conventions transformers produces:

* ``sdpa``-style masks: ``None`` without padding (the adapter then infers causal from
  ``module.is_causal``), a bool keep-mask ``[B, 1, T, T]`` with padding;
* ``eager``-style masks: an additive float mask (0 / large negative), which the
  adapter divides by ``scaling`` into a score (``attention_mask_is_scaled``).

Checks:
* every attention call inside the model matches the eager oracle
  (oracle/eager.py) run in fp32 on the CPU on the same q/k/v/mask, at the
  bf16 bar of the parity suite, on the rows that keep a key;
* the model's hidden states match HuggingFace's own eager attention run in fp32
  on the CPU with the same weights (cosine > 0.999 on non-padding tokens);
* without padding, a backward through the model gives finite gradients for every
  parameter.

With left padding, transformers' masks leave the padding query rows with no kept
key.  Under the eager semantics the build follows (the reference's eager
attention, benchmark/precision_check.py:133-180), such a row's output is NaN and the dV of its
kv-head is NaN; a NaN row then reaches the next layer as a masked key whose V is
NaN (0 x NaN = NaN in P V, in eager attention too).  The padding cases therefore
run one layer and check the forward only, on the non-padding tokens; padded
batches should be unpadded or passed without padding (README.md:73-77).
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")


def _model(attn, layers, head_dim=64):
    from transformers import LlamaConfig, LlamaModel

    cfg = LlamaConfig(vocab_size=128, hidden_size=256, intermediate_size=512, num_hidden_layers=layers,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=head_dim, max_position_embeddings=512,
                      attn_implementation=attn)
    torch.manual_seed(0)
    return LlamaModel(cfg)


def _register(name, mask_fn, records):
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface

    import tilelang_fa2_4d_mask as api
    from oracle import eager as E

    def attn(module, query, key, value, attention_mask, scaling, dropout=0.0, **kwargs):
        out, w = api.tilelang_attention_forward(module, query, key, value, attention_mask, scaling, dropout, **kwargs)
        assert w is None and out.shape == query.shape
        # oracle on the same inputs, the way the adapter interprets them
        mask = score = None
        causal = attention_mask is None and bool(module.is_causal)
        if attention_mask is not None:
            if attention_mask.dtype == torch.bool:
                mask = attention_mask.detach().cpu()
            else:
                score = attention_mask.detach().float().cpu() / scaling
        ref = E.eager_ref(query.detach().float().cpu(), key.detach().float().cpu(),
                                value.detach().float().cpu(), mask, score, scale=scaling, is_causal=causal)
        records.append((out.detach().float().cpu(), ref))
        return out.transpose(1, 2).contiguous(), None   # HF expects [B, T, H, D]

    AttentionInterface.register(name, attn)
    AttentionMaskInterface.register(name, mask_fn)


@pytest.mark.parametrize("head_dim", [64, 256])
@pytest.mark.parametrize("style", ["sdpa", "eager"])
@pytest.mark.parametrize("padding", [False, True], ids=["nopad", "leftpad"])
def test_llama_with_fa2_attention(cuda, style, padding, head_dim):
    from transformers.masking_utils import eager_mask, sdpa_mask

    name = f"tilelang_fa2_{style}"
    records = []
    _register(name, sdpa_mask if style == "sdpa" else eager_mask, records)
    print(f"case llama {style} masks, padding={padding}, head_dim={head_dim}", flush=True)

    layers = 1 if padding else 2
    ours = _model(name, layers, head_dim).to(device=cuda, dtype=torch.bfloat16)
    ref = _model("eager", layers, head_dim)
    ref.load_state_dict({k: v.float().cpu() for k, v in ours.state_dict().items()})
    ref.eval()
    ours.eval()

    g = torch.Generator().manual_seed(1)
    T = 96
    ids = torch.randint(0, 128, (2, T), generator=g)
    am = torch.ones(2, T, dtype=torch.long)
    if padding:
        am[1, :7] = 0
    keep_tok = am.bool()

    h = ours(input_ids=ids.to(cuda), attention_mask=am.to(cuda)).last_hidden_state
    assert len(records) == layers   # one attention call per layer
    for out, r in records:
        rows_ok = torch.isfinite(r).all(-1)   # rows that keep a key (padding queries may keep none)
        err = (out - r).abs()[rows_ok]
        print(f"  attention call: max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}", flush=True)
        assert (err <= 2e-2 + 2.0 ** -6 * r.abs()[rows_ok]).all()
        assert err.mean().item() <= max(1e-4, 2.0 ** -8 * r.abs()[rows_ok].mean().item())

    with torch.no_grad():
        h_ref = ref(input_ids=ids, attention_mask=am).last_hidden_state
    a = h.detach().float().cpu()[keep_tok]
    b = h_ref[keep_tok]
    cos = torch.nn.functional.cosine_similarity(a, b, dim=-1)
    print(f"  hidden states vs HF eager fp32: min cosine {cos.min().item():.6f}", flush=True)
    assert cos.min().item() > 0.999

    if padding:
        return
    # backward through the model
    ours.train()
    records.clear()
    h = ours(input_ids=ids.to(cuda), attention_mask=am.to(cuda)).last_hidden_state
    (h.float()[keep_tok.to(cuda)] ** 2).mean().backward()
    for n, p in ours.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all(), n


@pytest.mark.parametrize("atomic", [True, False], ids=["atomic", "det"])
def test_eager_style_padding_backward(cuda, atomic):
    """One attention layer's forward and backward under transformers' eager-style
    mask with left padding: causal + padding as an additive bf16 mask (0 or
    finfo(bf16).min), [B, 1, T, T], through ``tilelang_attention_forward``.  The
    adapter divides it by ``scaling`` (attention_mask_is_scaled), which overflows
    to -inf in fp32 (python/modeling_attention.py:129-133), so the padding query
    rows have every logit -inf: eager autograd gives them a NaN output row and a
    NaN dQ row, NaN dK and dV for every key of their kv-heads (no key is dropped
    by a bool mask or by causality here, the mask being additive).  Checked
    against the oracle (autograd through the eager graph, fp32, CPU) with NaN
    positions compared exactly."""
    import tilelang_fa2_4d_mask as api
    from oracle import eager as E

    B, H, Hk, T, D = 2, 4, 2, 96, 64
    pad = 7
    g = torch.Generator().manual_seed(3)
    q = torch.randn((B, H, T, D), generator=g).to(torch.bfloat16)
    k = torch.randn((B, Hk, T, D), generator=g).to(torch.bfloat16)
    v = torch.randn((B, Hk, T, D), generator=g).to(torch.bfloat16)
    do = torch.randn((B, H, T, D), generator=g).to(torch.bfloat16)
    keep = torch.ones((B, 1, T, T), dtype=torch.bool).tril()
    keep[1, :, :, :pad] = False                    # left padding of sequence 1 (keys)
    am = torch.zeros((B, 1, T, T), dtype=torch.bfloat16).masked_fill(~keep, torch.finfo(torch.bfloat16).min)
    scaling = D ** -0.5
    assert torch.isinf(am.float() / scaling).any()   # the overflow this case is about

    class _Attn(torch.nn.Module):
        is_causal = True

    qd, kd, vd = (t.to(cuda).requires_grad_(True) for t in (q, k, v))
    print(f"case eager-style padding backward atomic={atomic}", flush=True)
    out, w = api.tilelang_attention_forward(_Attn(), qd, kd, vd, am.to(cuda), scaling, use_atomic_backward=atomic)
    out.backward(do.to(cuda))
    torch.cuda.synchronize()
    ours = {"out": out.detach().float().cpu(), "dq": qd.grad.float().cpu(), "dk": kd.grad.float().cpu(),
            "dv": vd.grad.float().cpu()}
    o, dq, dk, dv = E.eager_fwd_bwd(q, k, v, None, am.float() / scaling, do, scale=scaling, is_causal=False)
    ref = {"out": o.float(), "dq": dq.float(), "dk": dk.float(), "dv": dv.float()}
    assert torch.isnan(ref["dq"][1, :, :pad]).all() and torch.isnan(ref["dk"][1]).all()
    for name in ref:
        st = E.finite_diff_stats(ours[name], ref[name])
        r = ref[name]
        fin = torch.isfinite(r)
        print(f"  {name}: max_abs={st['max_abs']:.3e} mean_abs={st['mean_abs']:.3e} nan_match={st['nan_match']}",
              flush=True)
        assert st["nan_match"], name
        if fin.any():
            err = (ours[name][fin] - r[fin]).abs()
            assert (err <= 2e-2 + 2.0 ** -6 * r[fin].abs()).all(), name
            assert err.mean().item() <= max(1e-4, 2.0 ** -8 * r[fin].abs().mean().item()), name
