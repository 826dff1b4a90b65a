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
    np_ = m["Bm"] * m["Hm"]
    m["bits"] = 0
    m["bitsT"] = a256(np_ * m["pbits"])
    m["blk"] = a256(m["bitsT"] + np_ * m["pbitsT"])
    m["lfwd"] = a256(m["blk"] + np_ * m["pblk"])
    m["lkv"] = a256(m["lfwd"] + np_ * m["plfwd"])
    m["ldq"] = a256(m["lkv"] + np_ * m["plkv"])
    m["ord"] = a256(m["ldq"] + np_ * m["pldq"])
    m["total"] = a256(m["ord"] + np_ * m["pord"])
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
