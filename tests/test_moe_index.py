"""Host emulation of the routed MoE's device index math (no GPU).

Restates, from plugins_amd/csrc/exl3_kernels.hip and exl3_kern.h, what the
routed SwiGLU's kernels address at the DeepSeek-V3 shape (hidden 7168,
expert intermediate 2048, 256 experts, top-8, K = 3) for prefill-sized
batches up to 2048 tokens (16384 slots):

* moe_route_kernel: per-expert counts, the slots sorted by expert (exclusive
  scan offsets), work items of at most `item_rows` slots of one expert;
* gemm_grouped_kernel: the activation rows it gathers (the direct LDS loads'
  32-bit byte offsets), the trellis words its decode waves read, the output
  rows it scatters to;
* moe_gemv_kernel: the rows, outputs and partial-sum slots of its items.

Every address is checked against the size of the buffer it indexes, as
moe_layout sizes them.  The routings are the bench's (softmax of N(0,1)
logits, top-8) plus adversarial ones: every slot on one expert, and slot
counts that are multiples of the item size plus one.
"""
import numpy as np
import pytest

E, HIDDEN, INTER, TOPK, K = 256, 7168, 2048, 8, 3
GM_BM, MOE_ITEM_ROWS = 256, 4


def route(inds: np.ndarray, experts: int, item_rows: int):
    """moe_route_kernel: (sorted slots, items [(expert, start, count)])."""
    flat = inds.reshape(-1).astype(np.int64)
    valid = flat < experts
    cnt = np.bincount(flat[valid], minlength=experts)
    off = np.concatenate([[0], np.cumsum(cnt)[:-1]])
    # slots of an expert in any order (the kernel's atomics); slot order here
    order = np.argsort(np.where(valid, flat, experts), kind="stable")[: valid.sum()]
    sorted_slots = order.astype(np.int64)
    assert np.array_equal(np.sort(flat[sorted_slots]), flat[sorted_slots])
    items = []
    for e in range(experts):
        c = int(cnt[e])
        for r in range((c + item_rows - 1) // item_rows):
            items.append((e, int(off[e]) + r * item_rows, min(item_rows, c - r * item_rows)))
    return sorted_slots, items, cnt


def max_items(experts: int, slots: int, item_rows: int) -> int:
    """moe_layout's bound on the item count (the grid's item dimension)."""
    return min(experts, slots) + (slots + item_rows - 1) // item_rows


def check_grouped_gemm(sorted_slots, items, slots, in_f, out_f, n, experts):
    """gemm_grouped_kernel over every item: returns the largest byte offset
    of the activation loads, the largest trellis dword and output element."""
    in_tiles, out_tiles = in_f // 16, out_f // 16
    k = n // 16
    NW = 8 * k
    NS = in_tiles // 4
    assert NS % 2 == 0 and NS >= 2, "gw_mfma_main takes an even stage count"
    expert_words = in_tiles * out_tiles * n // 2
    wstage = 4 * out_tiles * NW
    lane = np.arange(64)
    max_act = max_tw = max_out = 0
    for (e, start, M) in items:
        assert 1 <= M <= GM_BM and start + M <= len(sorted_slots)
        rows = sorted_slots[start + np.minimum(np.arange(GM_BM), M - 1)]
        # MFMA waves 0-7: rows 32 w + 8 u + l / 8, piece (l % 8) ^ ((R / 2) % 8),
        # then the stage's base st * 128 bytes and the 16 bytes of the load
        for w in range(8):
            for u in range(4):
                R = 32 * w + 8 * u + (lane >> 3)
                q = (lane & 7) ^ ((R >> 1) & 7)
                voff = (rows[R] * in_f + 8 * q) * 2
                assert voff.max() < 2 ** 32, "32-bit activation offset overflows"
                max_act = max(max_act, int(voff.max()) + (NS - 1) * 128 + 16)
        # decode waves: chunk c of tile tnl of k-tile row tkl, K words per stage
        cgs = out_tiles // 8
        dt = np.arange(256)
        tkl, tnl, c = dt >> 6, (dt >> 3) & 7, dt & 7
        for cg in (0, cgs - 1):
            twc = e * expert_words + (tkl * out_tiles + cg * 8 + tnl) * NW + c * k
            last = twc + (NS - 1) * wstage + (k - 1)
            max_tw = max(max_tw, int(last.max()))
            assert twc.min() >= e * expert_words
            # the history word comes from lane c - 1 of the same tile
            assert np.all(((lane & ~7) | ((lane + 7) & 7)) // 8 == lane // 8)
            # outputs: rows orow(m) = rows[m], m < M, columns cg * 128 + 0..127
            max_out = max(max_out, int(rows[:M].max()) * out_f + cg * 128 + 127)
    assert max_act <= slots * in_f * 2, (max_act, slots * in_f * 2)
    assert max_tw < experts * expert_words
    assert max_out < slots * out_f
    return max_act, max_tw, max_out


def routings(rng, tokens):
    probs = rng.standard_normal((tokens, E))
    top = np.argsort(-probs, axis=1)[:, :TOPK].astype(np.int32)
    yield "softmax top-8", top
    yield "one expert", np.zeros((tokens, TOPK), np.int32) + 7
    # every expert 256 k + 1 slots where possible (one item of one slot each)
    flat = np.repeat(np.arange(E, dtype=np.int32), (tokens * TOPK) // E + 1)[: tokens * TOPK]
    yield "even plus one", flat.reshape(tokens, TOPK)
    # out-of-range experts contribute nothing
    bad = top.copy()
    bad[:, 0] = E + 3
    yield "out of range", bad


@pytest.mark.parametrize("tokens", [256, 1024, 2048])
def test_grouped_gemm_indices_deepseek_v3(tokens):
    rng = np.random.default_rng(tokens)
    slots = tokens * TOPK
    assert slots <= 65535, "launch_moe refuses more slots"
    assert slots * max(HIDDEN, INTER) < 2 ** 31
    for name, inds in routings(rng, tokens):
        sorted_slots, items, cnt = route(inds, E, GM_BM)
        assert len(items) <= max_items(E, slots, GM_BM), name
        assert len(sorted_slots) == int(cnt.sum()) <= slots
        # gate / up: 7168 -> 2048 on the per-slot prepared rows (xg, xu: one
        # row per slot); down: 2048 -> 7168 on xd (one row per slot)
        check_grouped_gemm(sorted_slots, items, slots, HIDDEN, INTER, 16 * K, E)
        check_grouped_gemm(sorted_slots, items, slots, INTER, HIDDEN, 16 * K, E)


@pytest.mark.parametrize("tokens", [1, 16, 64, 2048])
def test_routed_gemv_items_deepseek_v3(tokens):
    """moe_gemv_kernel's items of up to 4 slots: rows, outputs and the
    partial-sum rows stay inside slots x width."""
    rng = np.random.default_rng(1 + tokens)
    slots = tokens * TOPK
    for name, inds in routings(rng, tokens):
        sorted_slots, items, _ = route(inds, E, MOE_ITEM_ROWS)
        assert len(items) <= max_items(E, slots, MOE_ITEM_ROWS), name
        for (e, start, count) in items:
            assert 1 <= count <= MOE_ITEM_ROWS
            b = np.minimum(np.arange(16), count - 1)
            slot = sorted_slots[start + b]
            # raw gate/up inputs are rows slot / topk of x; outputs rows slot
            assert (slot // TOPK).max() < tokens
            assert slot.max() * INTER + INTER <= slots * INTER
            assert slot.max() * HIDDEN + HIDDEN <= slots * HIDDEN
