"""GPU test of the mask preparation (fa_mask_prepare): the workspace the
attention kernels read -- bits, transposed bits, 32x32 block states and the
three live-tile lists -- decoded here and compared, bit for bit, with a torch
restatement of their definitions (include/fa2_4d_mask.h, MaskLayout in
csrc/fa_kernels.h).  Shapes cover ragged Tq/Tk, batch/head broadcast (stride
0), causal and non-causal, all-true / all-false / packed-document masks.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

FWD_ROWS, FWD_KEYS, KV_KEYS, DQ_ROWS = 256, 64, 128, 256


def cdiv(a, b):
    return (a + b - 1) // b


def layout(B, Hq, Tq, Tk, bcast_b, bcast_h):
    """Byte offsets of the workspace arrays (same rules as mask_layout)."""
    a256 = lambda x: (x + 255) & ~255  # noqa: E731
    m = dict(Bm=1 if bcast_b else B, Hm=1 if bcast_h else Hq, nq32=cdiv(Tq, 32), nk32=cdiv(Tk, 32))
    m["wk"] = (m["nk32"] + 3) & ~3
    m["wq"] = (m["nq32"] + 3) & ~3
    m["nfq"], m["nft"] = cdiv(Tq, FWD_ROWS), cdiv(Tk, FWD_KEYS)
    m["nkb"], m["ndq"] = cdiv(Tk, KV_KEYS), cdiv(Tq, DQ_ROWS)
    m["pbits"] = Tq * m["wk"] * 4
    m["pbitsT"] = m["nk32"] * m["wq"] * 32 * 4
    m["pblk"] = m["nq32"] * m["nk32"]
    m["plfwd"] = m["nfq"] * (1 + m["nft"]) * 4
    m["plkv"] = m["nkb"] * (1 + m["nq32"]) * 4
    m["pldq"] = m["ndq"] * (1 + m["nk32"]) * 4
    m["pord"] = (m["nfq"] + m["nkb"] + m["ndq"]) * 4
    m["phist"] = (m["nft"] + 1 + m["nq32"] + 1 + m["nk32"] + 1) * 4
    np_ = m["Bm"] * m["Hm"]
    m["bits"] = 0
    m["bitsT"] = a256(np_ * m["pbits"])
    m["blk"] = a256(m["bitsT"] + np_ * m["pbitsT"])
    m["lfwd"] = a256(m["blk"] + np_ * m["pblk"])
    m["lkv"] = a256(m["lfwd"] + np_ * m["plfwd"])
    m["ldq"] = a256(m["lkv"] + np_ * m["plkv"])
    m["ord"] = a256(m["ldq"] + np_ * m["pldq"])
    m["hist"] = a256(m["ord"] + np_ * m["pord"])
    m["total"] = a256(m["hist"] + np_ * m["phist"])
    return m


def pack_bits(keep):
    """[R, C] bool -> [R, ceil(C/32)] int64 words, bit c%32 of word c/32."""
    R, C = keep.shape
    n = cdiv(C, 32)
    pad = torch.zeros((R, n * 32), dtype=torch.int64)
    pad[:, :C] = keep.long()
    w = pad.view(R, n, 32) << torch.arange(32, dtype=torch.int64)
    return w.sum(-1)


def expected(plane_mask, Tq, Tk, causal, m):
    """Expected arrays of one plane from its [Tq, Tk] bool mask."""
    keep = plane_mask
    bits = pack_bits(keep)                      # [Tq, nk32]
    bitsT = pack_bits(keep.t().contiguous())    # [Tk, nq32]: word i/32 of key j
    nq32, nk32 = m["nq32"], m["nk32"]
    blk = torch.zeros((nq32, nk32), dtype=torch.uint8)
    for rb in range(nq32):
        for kb in range(nk32):
            t = keep[32 * rb:32 * rb + 32, 32 * kb:32 * kb + 32]
            blk[rb, kb] = 0 if not bool(t.any()) else (2 if bool(t.all()) else 1)

    def fwd_list(qb):
        q_last = min(Tq - 1, FWD_ROWS * qb + FWD_ROWS - 1)
        out = []
        for t in range(m["nft"]):
            if causal and FWD_KEYS * t > q_last:
                continue
            sub = blk[8 * qb:8 * qb + 8, 2 * t:2 * t + 2]
            if bool((sub != 0).any()):
                out.append(t | (0x80000000 if bool((sub == 2).all()) else 0))
        return out

    def kv_list(kb):
        out = []
        for s in range(nq32):
            if causal and min(Tq - 1, 32 * s + 31) < KV_KEYS * kb:
                continue
            if bool((blk[s, 4 * kb:4 * kb + 4] != 0).any()):
                out.append(s)
        return out

    def dq_list(qb):
        q_last = min(Tq - 1, DQ_ROWS * qb + DQ_ROWS - 1)
        out = []
        for c in range(nk32):
            if causal and 32 * c > q_last:
                continue
            if bool((blk[8 * qb:8 * qb + 8, c] != 0).any()):
                out.append(c)
        return out

    return bits, bitsT, blk, [fwd_list(i) for i in range(m["nfq"])], [kv_list(i) for i in range(m["nkb"])], \
        [dq_list(i) for i in range(m["ndq"])]


def read_lists(ws32, off, n, width):
    lists = []
    base = off // 4
    for i in range(n):
        row = ws32[base + i * width: base + (i + 1) * width]
        cnt = int(row[0])
        lists.append([int(x) & 0xFFFFFFFF for x in row[1:1 + cnt]])
    return lists


def make_mask(kind, B, Hm, Tq, Tk, gen):
    if kind == "rand":
        return torch.rand((B, Hm, Tq, Tk), generator=gen) < 0.5
    if kind == "sparse":
        return torch.rand((B, Hm, Tq, Tk), generator=gen) < 0.002
    if kind == "ones":
        return torch.ones((B, Hm, Tq, Tk), dtype=torch.bool)
    if kind == "zeros":
        return torch.zeros((B, Hm, Tq, Tk), dtype=torch.bool)
    if kind == "docs":
        m = torch.zeros((B, Hm, Tq, Tk), dtype=torch.bool)
        for b in range(B):
            pos = 0
            while pos < min(Tq, Tk):
                n = int(torch.randint(20, 300, (1,), generator=gen))
                m[b, :, pos:pos + n, pos:pos + n] = True
                pos += n
        return m & torch.ones((Tq, Tk), dtype=torch.bool).tril()
    raise ValueError(kind)


CASES = [
    # B, Hq, mask heads, Tq, Tk, causal, kind
    (1, 2, 2, 256, 256, False, "rand"),
    (2, 3, 1, 300, 520, True, "rand"),
    (1, 4, 4, 77, 1000, False, "sparse"),
    (2, 2, 1, 1030, 700, True, "docs"),
    (1, 1, 1, 513, 513, False, "ones"),
    (1, 2, 1, 96, 33, True, "zeros"),
    (3, 2, 2, 200, 4100, False, "docs"),
]


@pytest.mark.parametrize("B,Hq,Hm,Tq,Tk,causal,kind", CASES)
def test_prepared_mask_matches_definition(cuda, B, Hq, Hm, Tq, Tk, causal, kind):
    from tilelang_fa2_4d_mask import fa2

    print(f"case B{B} Hq{Hq} Hm{Hm} Tq{Tq} Tk{Tk} causal={causal} {kind}", flush=True)
    gen = torch.Generator().manual_seed(Tq * 7 + Tk)
    bm = 1 if kind == "docs" and B > 1 and Hm == 1 and Tk > 4000 else B   # one batch-broadcast case
    mask = make_mask(kind, bm, Hm, Tq, Tk, gen)
    dev_mask = mask.to(cuda)
    view = dev_mask.expand(B, Hq, Tq, Tk)
    mst = fa2._norm_strides(view)[:3]
    ws = fa2._prepare_mask(view, mst, B, Hq, Tq, Tk, causal, cuda)
    torch.cuda.synchronize()
    m = layout(B, Hq, Tq, Tk, mst[0] == 0, mst[1] == 0)
    assert ws.numel() == m["total"]
    ws_cpu = ws.cpu()
    ws32 = ws_cpu[: m["total"] // 4 * 4].view(torch.int32)
    for pm in range(m["Bm"] * m["Hm"]):
        bb, hh = divmod(pm, m["Hm"])
        bits, bitsT, blk, lf, lk, ld = expected(mask[min(bb, bm - 1), hh], Tq, Tk, causal, m)
        got_bits = ws32[(m["bits"] + pm * m["pbits"]) // 4:][: Tq * m["wk"]].view(Tq, m["wk"]).long() & 0xFFFFFFFF
        assert torch.equal(got_bits[:, : m["nk32"]], bits), f"bits plane {pm}"
        assert not got_bits[:, m["nk32"]:].any(), "padding words"
        # [nk32][wq][32 keys] -> [key][word]
        got_t = ws32[(m["bitsT"] + pm * m["pbitsT"]) // 4:][: m["nk32"] * m["wq"] * 32]
        got_t = got_t.view(m["nk32"], m["wq"], 32).permute(0, 2, 1).reshape(m["nk32"] * 32, m["wq"])[:Tk]
        assert torch.equal(got_t.long()[:, : m["nq32"]] & 0xFFFFFFFF, bitsT), f"bitsT plane {pm}"
        got_blk = ws_cpu[m["blk"] + pm * m["pblk"]:][: m["pblk"]].view(m["nq32"], m["nk32"])
        assert torch.equal(got_blk, blk), f"blk plane {pm}"
        assert read_lists(ws32, m["lfwd"] + pm * m["plfwd"], m["nfq"], 1 + m["nft"]) == lf, f"fwd lists plane {pm}"
        assert read_lists(ws32, m["lkv"] + pm * m["plkv"], m["nkb"], 1 + m["nq32"]) == lk, f"kv lists plane {pm}"
        assert read_lists(ws32, m["ldq"] + pm * m["pldq"], m["ndq"], 1 + m["nk32"]) == ld, f"dq lists plane {pm}"
        # units of each list kind by count, largest first, ties by unit
        got_ord = ws32[(m["ord"] + pm * m["pord"]) // 4:][: m["nfq"] + m["nkb"] + m["ndq"]].tolist()
        want_ord = []
        for lists in (lf, lk, ld):
            want_ord += sorted(range(len(lists)), key=lambda i: (-len(lists[i]), i))
        assert got_ord == want_ord, f"order plane {pm}"


def _pack_words(keep):
    """[..., C] bool -> [..., ceil(C/32)] int64 words (vectorised pack_bits)."""
    C = keep.shape[-1]
    n = cdiv(C, 32)
    pad = torch.zeros(keep.shape[:-1] + (n * 32,), dtype=torch.int64, device=keep.device)
    pad[..., :C] = keep.long()
    return (pad.view(keep.shape[:-1] + (n, 32)) << torch.arange(32, dtype=torch.int64, device=keep.device)).sum(-1)


def _check_bits_and_blocks(ws, mask, m, Tq, Tk):
    """bits, bitsT and block states of every plane (Tq, Tk multiples of 32)."""
    P = m["Bm"] * m["Hm"]
    planes = mask.reshape(P, Tq, Tk)
    ws32 = ws[: m["total"] // 4 * 4].view(torch.int32)
    got = ws32[m["bits"] // 4:][: P * Tq * m["wk"]].view(P, Tq, m["wk"]).long() & 0xFFFFFFFF
    assert torch.equal(got[:, :, : m["nk32"]], _pack_words(planes)), "bits"
    got_t = ws32[m["bitsT"] // 4:][: P * m["nk32"] * m["wq"] * 32].view(P, m["nk32"], m["wq"], 32)
    got_t = got_t.permute(0, 1, 3, 2).reshape(P, m["nk32"] * 32, m["wq"]).long() & 0xFFFFFFFF
    assert torch.equal(got_t[:, :Tk, : m["nq32"]], _pack_words(planes.transpose(1, 2).contiguous())), "bitsT"
    blocks = planes.view(P, m["nq32"], 32, m["nk32"], 32)
    want = torch.where(blocks.any(4).any(2), torch.where(blocks.all(4).all(2), 2, 1), 0).to(torch.uint8)
    got_b = ws[m["blk"]:][: P * m["pblk"]].view(P, m["nq32"], m["nk32"])
    assert torch.equal(got_b, want), "blk"


def _attention_vs_oracle(q, k, v, mask, do, label, long_sums=False, causal=False):
    """fwd+bwd in both modes against the eager oracle (small-shape bar per
    entry, met against eager or against the rounding restatement, which
    makes the reference kernel's 16-bit roundings of P and dS,
    python/fa2.py:128-129, 287, 291: with millions of rows of at most 64 keys
    a few early causal rows sit where those roundings alone miss the bar;
    mean against eager).
    long_sums: dK / dV entries sum millions of products of 16-bit-rounded dS
    and P, whose error is that rounding's random walk, ~2^-9 of the entries'
    typical size whatever an entry's own value: their absolute term scales
    with mean |ref| then."""
    import tilelang_fa2_4d_mask as api
    from oracle import eager as E
    from oracle import rounding as R

    ref = E.eager_grads_chunked(q, k, v, mask, None, do, scale=q.shape[-1] ** -0.5, is_causal=causal,
                                block=65536)
    rr = R.rounded_attention(q, k, v, mask, None, do, scale=q.shape[-1] ** -0.5, is_causal=causal,
                             round_dtype=q.dtype, block=65536)
    for atomic in (True, False):
        qq, kk, vv = (x.detach().requires_grad_(True) for x in (q, k, v))
        out = api.tilelang_flash_attention(qq, kk, vv, mask=mask, is_causal=causal, use_atomic_backward=atomic)
        out.backward(do)
        torch.cuda.synchronize()
        for name, a, r in zip(("out", "dq", "dk", "dv"), (out, qq.grad, kk.grad, vv.grad), ref):
            a, r, rd = a.float(), r.float(), rr[name].float()
            assert torch.equal(torch.isnan(a), torch.isnan(r)), f"{label} {name}: NaN positions"
            fin = torch.isfinite(r)
            err = (a[fin] - r[fin]).abs()
            print(f"[{label} atomic={atomic}] {name}: max={err.max().item():.3e} mean={err.mean().item():.3e}",
                  flush=True)
            floor = 2.0 ** -6 * r[fin].abs().mean().item() if long_sums and name in ("dk", "dv") else 2e-2
            off_eager = err > floor + 2.0 ** -6 * r[fin].abs()
            off_rounded = (a[fin] - rd[fin]).abs() > floor + 2.0 ** -6 * rd[fin].abs()
            assert not bool((off_eager & off_rounded).any()), f"{label} {name}"
            assert err.mean().item() <= max(1e-4, 2.0 ** -8 * r[fin].abs().mean().item()), f"{label} {name}"


@pytest.mark.parametrize("causal", [False, True], ids=["noncausal", "causal"])
def test_more_planes_than_one_grid_dimension(cuda, causal):
    """A per-head mask of 2100 x 32 = 67200 planes: more than the 65535 a grid
    dimension holds, so the preparation walks its planes with a grid stride
    (large batches of short sequences reach this)."""
    from tilelang_fa2_4d_mask import fa2

    B, H, T, D = 2100, 32, 64, 64
    print(f"case B{B} H{H} T{T} D{D} per-head mask: {B * H} planes, causal={causal}", flush=True)
    g = torch.Generator(device=cuda).manual_seed(11)
    mask = torch.rand((B, H, T, T), generator=g, device=cuda) < 0.6
    mask[:, :, torch.arange(T), torch.arange(T)] = True
    mst = fa2._norm_strides(mask)[:3]
    ws = fa2._prepare_mask(mask, mst, B, H, T, T, causal, cuda)
    torch.cuda.synchronize()
    m = layout(B, H, T, T, False, False)
    assert ws.numel() == m["total"]
    _check_bits_and_blocks(ws, mask, m, T, T)
    # lists and order of the first and last planes against the definition
    ws_cpu = ws.cpu()
    ws32 = ws_cpu[: m["total"] // 4 * 4].view(torch.int32)
    for pm in (0, B * H - 1):
        _, _, _, lf, lk, ld = expected(mask[pm // H, pm % H].cpu(), T, T, causal, m)
        assert read_lists(ws32, m["lfwd"] + pm * m["plfwd"], m["nfq"], 1 + m["nft"]) == lf, f"fwd lists {pm}"
        assert read_lists(ws32, m["lkv"] + pm * m["plkv"], m["nkb"], 1 + m["nq32"]) == lk, f"kv lists {pm}"
        assert read_lists(ws32, m["ldq"] + pm * m["pldq"], m["ndq"], 1 + m["nk32"]) == ld, f"dq lists {pm}"
    rnd = lambda *s: torch.randn(s, generator=g, device=cuda).to(torch.bfloat16)  # noqa: E731
    _attention_vs_oracle(rnd(B, H, T, D), rnd(B, H, T, D), rnd(B, H, T, D), mask, rnd(B, H, T, D), "planes",
                         causal=causal)


@pytest.mark.parametrize("causal", [False, True], ids=["noncausal", "causal"])
def test_more_row_blocks_than_one_grid_dimension(cuda, causal):
    """Tq 2^21 + 64: 65538 blocks of 32 rows, past the 65535 of a grid
    dimension, so the preparation walks its row blocks with a grid stride."""
    from tilelang_fa2_4d_mask import fa2

    Tq, Tk, D = (1 << 21) + 64, 64, 64
    print(f"case B1 H1 Tq{Tq} Tk{Tk} D{D}: {Tq // 32} row blocks, causal={causal}", flush=True)
    g = torch.Generator(device=cuda).manual_seed(12)
    mask = torch.rand((1, 1, Tq, Tk), generator=g, device=cuda) < 0.5
    mask[:, :, :, 0] = True
    mst = fa2._norm_strides(mask)[:3]
    ws = fa2._prepare_mask(mask, mst, 1, 1, Tq, Tk, causal, cuda)
    torch.cuda.synchronize()
    m = layout(1, 1, Tq, Tk, True, True)
    assert ws.numel() == m["total"]
    _check_bits_and_blocks(ws, mask, m, Tq, Tk)
    rnd = lambda *s: torch.randn(s, generator=g, device=cuda).to(torch.bfloat16)  # noqa: E731
    _attention_vs_oracle(rnd(1, 1, Tq, D), rnd(1, 1, Tk, D), rnd(1, 1, Tk, D), mask, rnd(1, 1, Tq, D), "rows",
                         long_sums=True, causal=causal)
