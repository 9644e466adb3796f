"""The Qwen3-8B-shaped decode step around the EXL3 linears.

The harness ops (include/exl3_decoder.h) are floating-point kernels, so each
is checked against a float32 PyTorch restatement of the same op (on the CPU,
so no library product is involved), with the tolerance written at each check;
the whole step is checked against a float32 restatement whose linears are the
library's EXL3 matmuls (those are pinned to the oracle in test_gpu_parity.py),
so the comparison isolates norm, RoPE, KV append, attention and SwiGLU."""
import math
import os
import re

import numpy as np
import pytest

from plugins_amd import exl3 as X

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_decoder_header_symbols_are_exported():
    from plugins_amd import qwen3 as Q
    text = open(os.path.join(ROOT, "include", "exl3_decoder.h")).read()
    declared = set(re.findall(r"\b(exl3d_[a-z_0-9]+)\s*\(", text))
    L = X.lib()
    for name in sorted(declared):
        assert hasattr(L, name), name
    assert declared == set(Q._DEC_SIGS), declared ^ set(Q._DEC_SIGS)


# ------------------------------------------------------------- GPU parity

torch = pytest.importorskip("torch")
gpu = pytest.mark.gpu


def rel(a, b):
    a = a.double()
    b = b.double()
    return float((a - b).norm() / b.norm())


def ref_rmsnorm(h, w, eps):
    return (h * torch.rsqrt((h * h).mean(-1, keepdim=True) + eps) * w.float()).half()


def ref_qk_norm_rope(x, w, pos, eps, theta):
    """x [B, heads, 128] f16 -> f16: RMSNorm (rounded to f16), rotate-half RoPE."""
    n = ref_rmsnorm(x.float(), w, eps).float()
    i = torch.arange(64, dtype=torch.float32)
    inv = theta ** (-2.0 * i / 128.0)
    ang = pos.float()[:, None, None] * inv
    c, s = torch.cos(ang), torch.sin(ang)
    x1, x2 = n[..., :64], n[..., 64:]
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], -1).half()


def ref_attention(q, kc, vc, pos):
    """q [B, nq*128] f16, caches [B, nkv, T, 128] -> [B, nq*128] f16 (float32)."""
    B = q.shape[0]
    nkv = kc.shape[1]
    nq = q.shape[1] // 128
    out = torch.empty(B, nq * 128, dtype=torch.float16)
    for b in range(B):
        L = int(pos[b]) + 1
        K = kc[b, :, :L].float().repeat_interleave(nq // nkv, 0)
        V = vc[b, :, :L].float().repeat_interleave(nq // nkv, 0)
        Q = q[b].view(nq, 1, 128).float()
        p = torch.softmax((Q @ K.transpose(1, 2).contiguous()) / math.sqrt(128), -1)
        out[b] = (p @ V).view(-1).half()
    return out


@gpu
def test_embed_and_add_rmsnorm():
    from plugins_amd import qwen3 as Q
    g = torch.Generator().manual_seed(1)
    B, H, V = 5, 1024, 300
    table = torch.randn(V, H, generator=g).half()
    ids = torch.tensor([3, 0, 299, 17, 3], dtype=torch.int32)
    h = torch.empty(B, H, device="cuda")
    Q.embed(ids.cuda(), table.cuda(), h)
    assert torch.equal(h.cpu(), table[ids.long()].float())  # exact: f16 -> f32
    add = torch.randn(B, H, generator=g).half()
    w = (1 + 0.1 * torch.randn(H, generator=g)).half()
    out = torch.empty(B, H, dtype=torch.float16, device="cuda")
    Q.add_rmsnorm(h, add.cuda(), w.cuda(), out, 1e-6)
    href = table[ids.long()].float() + add.float()
    assert torch.allclose(h.cpu(), href, rtol=0, atol=0)  # one f32 add per element
    want = ref_rmsnorm(href, w, 1e-6)
    # f16 output: within one f16 rounding of the float32 reference
    assert rel(out.cpu(), want) < 2e-3, rel(out.cpu(), want)


@gpu
def test_qk_norm_rope_and_kv_append():
    from plugins_amd import qwen3 as Q
    g = torch.Generator().manual_seed(2)
    B, nq, nkv, T = 3, 8, 2, 64
    q = torch.randn(B, nq * 128, generator=g).half()
    k = torch.randn(B, nkv * 128, generator=g).half()
    v = torch.randn(B, nkv * 128, generator=g).half()
    qn = (1 + 0.1 * torch.randn(128, generator=g)).half()
    kn = (1 + 0.1 * torch.randn(128, generator=g)).half()
    pos = torch.tensor([0, 17, 63], dtype=torch.int32)
    kc = torch.zeros(B, nkv, T, 128, dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    qo = torch.empty(B, nq * 128, dtype=torch.float16, device="cuda")
    Q.qk_norm_rope(q.cuda(), k.cuda(), v.cuda(), qn.cuda(), kn.cuda(), pos.cuda(), qo, kc, vc, 1e-6,
                   1e6)
    wq = ref_qk_norm_rope(q.view(B, nq, 128), qn, pos, 1e-6, 1e6).view(B, -1)
    wk = ref_qk_norm_rope(k.view(B, nkv, 128), kn, pos, 1e-6, 1e6)
    # f16 outputs of a float32 computation (sincos / powf in f32): 2e-3 relative
    assert rel(qo.cpu(), wq) < 2e-3, rel(qo.cpu(), wq)
    kcc, vcc = kc.cpu(), vc.cpu()
    for b in range(B):
        p = int(pos[b])
        assert rel(kcc[b, :, p], wk[b]) < 2e-3
        assert torch.equal(vcc[b, :, p], v[b].view(nkv, 128))  # copied
        others = torch.ones(T, dtype=torch.bool)
        others[p] = False
        assert not kcc[b, :, others].any() and not vcc[b, :, others].any()  # only row pos written


@gpu
@pytest.mark.parametrize("B,T,lens", [(1, 40, [39]), (3, 2100, [2048, 5, 700]), (16, 300, None)])
def test_attention_decode(B, T, lens):
    from plugins_amd import qwen3 as Q
    g = torch.Generator().manual_seed(3 + B)
    nq, nkv = 32, 8
    q = torch.randn(B, nq * 128, generator=g).half()
    kc = torch.randn(B, nkv, T, 128, generator=g).half()
    vc = torch.randn(B, nkv, T, 128, generator=g).half()
    pos = torch.tensor(lens if lens else [int(x) for x in torch.randint(0, T, (B,), generator=g)],
                       dtype=torch.int32)
    out = torch.empty(B, nq * 128, dtype=torch.float16, device="cuda")
    scratch = torch.zeros(Q.attn_scratch_bytes(B, nq, nkv, T) // 4 + 1, device="cuda")
    want = ref_attention(q, kc, vc, pos)
    for _ in range(2):  # the second call reuses the scratch (its tickets were left zero)
        out.fill_(float("nan"))
        Q.attn_decode(q.cuda(), kc.cuda(), vc.cuda(), pos.cuda(), out, scratch)
        # f32 online softmax in another summation order, f16 output: 2e-3 relative
        assert rel(out.cpu(), want) < 2e-3, rel(out.cpu(), want)


@gpu
@pytest.mark.parametrize("B,T,lens", [(1, 80, [79]), (3, 2100, [2048, 5, 700]), (16, 300, None)])
def test_attention_decode_with_rope_and_append(B, T, lens):
    # q/k norm + RoPE + KV append + attention in one launch, against the
    # float32 restatement of the two steps
    from plugins_amd import qwen3 as Q
    g = torch.Generator().manual_seed(30 + B)
    nq, nkv = 32, 8
    q = torch.randn(B, nq * 128, generator=g).half()
    k = torch.randn(B, nkv * 128, generator=g).half()
    v = torch.randn(B, nkv * 128, generator=g).half()
    qn = (1 + 0.1 * torch.randn(128, generator=g)).half()
    kn = (1 + 0.1 * torch.randn(128, generator=g)).half()
    kc = torch.randn(B, nkv, T, 128, generator=g).half()
    vc = torch.randn(B, nkv, T, 128, generator=g).half()
    pos = torch.tensor(lens if lens else [int(x) for x in torch.randint(0, T, (B,), generator=g)],
                       dtype=torch.int32)
    kcd, vcd = kc.cuda(), vc.cuda()
    out = torch.empty(B, nq * 128, dtype=torch.float16, device="cuda")
    scratch = torch.zeros(Q.attn_scratch_bytes(B, nq, nkv, T) // 4 + 1, device="cuda")
    Q.attn_decode_rope(q.cuda(), k.cuda(), v.cuda(), qn.cuda(), kn.cuda(), pos.cuda(), kcd, vcd, out,
                       scratch, 1e-6, 1e6)
    wq = ref_qk_norm_rope(q.view(B, nq, 128), qn, pos, 1e-6, 1e6).view(B, -1)
    wk = ref_qk_norm_rope(k.view(B, nkv, 128), kn, pos, 1e-6, 1e6)
    kw, vw = kc.clone(), vc.clone()
    for b in range(B):
        kw[b, :, int(pos[b])] = wk[b]
        vw[b, :, int(pos[b])] = v[b].view(nkv, 128)
    kcc, vcc = kcd.cpu(), vcd.cpu()
    # the appended key: f16 outputs of a float32 computation, 2e-3 relative;
    # the value is copied; every other row is untouched
    for b in range(B):
        p = int(pos[b])
        assert rel(kcc[b, :, p], wk[b]) < 2e-3
        assert torch.equal(vcc[b, :, p], v[b].view(nkv, 128))
        others = torch.ones(T, dtype=torch.bool)
        others[p] = False
        assert torch.equal(kcc[b, :, others], kc[b, :, others])
        assert torch.equal(vcc[b, :, others], vc[b, :, others])
    want = ref_attention(wq, kw, vw, pos)
    assert rel(out.cpu(), want) < 2e-3, rel(out.cpu(), want)


def _ssq(h):
    """Sums of squares per 128 columns of an f32 [B, H] residual."""
    return (h.double() ** 2).view(h.shape[0], -1, 128).sum(-1).float()


@gpu
@pytest.mark.parametrize("B,T,lens", [(1, 2048, [2047]), (1, 80, [40]), (1, 20000, [19999]),
                                      (2, 300, [299, 7]), (16, 300, None)])
def test_attention_o_fused_equals_separate(B, T, lens):
    # exl3d_attn_o against its two steps (attention with its combine launch,
    # then the o linear with the residual finish): at rows in one prepare
    # batch o's prepare combines the key splits itself (with 96 splits at
    # T = 20000: two chunks of the split loop), above it the steps run as
    # they are; residual and its sums of squares equal bit for bit
    from plugins_amd import qwen3 as Q
    g = torch.Generator().manual_seed(60 + B + T)
    nq, nkv = 32, 8
    lo = Q.random_linear(torch, nq * 128, 4096, 4, torch.Generator(device="cuda").manual_seed(7))
    q = torch.randn(B, nq * 128, generator=g).half().cuda()
    k = torch.randn(B, nkv * 128, generator=g).half().cuda()
    v = torch.randn(B, nkv * 128, generator=g).half().cuda()
    qn = (1 + 0.1 * torch.randn(128, generator=g)).half().cuda()
    kn = (1 + 0.1 * torch.randn(128, generator=g)).half().cuda()
    kc = torch.randn(B, nkv, T, 128, generator=g).half().cuda()
    vc = torch.randn(B, nkv, T, 128, generator=g).half().cuda()
    pos = torch.tensor(lens if lens else [int(x) for x in torch.randint(0, T, (B,), generator=g)],
                       dtype=torch.int32).cuda()
    h = torch.randn(B, 4096, generator=g).cuda()
    scratch = torch.zeros(Q.attn_scratch_bytes(B, nq, nkv, T) // 4 + 1, device="cuda")
    # the two steps
    kc1, vc1, h1 = kc.clone(), vc.clone(), h.clone()
    att1 = torch.empty(B, nq * 128, dtype=torch.float16, device="cuda")
    ssq1 = torch.empty(B, 32, device="cuda")
    Q.attn_decode_rope(q, k, v, qn, kn, pos, kc1, vc1, att1, scratch, 1e-6, 1e6)
    Q.linears([lo.weight], att1, res=h1, res_ssq=ssq1)
    # the fused entry
    kc2, vc2, h2 = kc.clone(), vc.clone(), h.clone()
    att2 = torch.empty(B, nq * 128, dtype=torch.float16, device="cuda")
    ssq2 = torch.empty(B, 32, device="cuda")
    scratch.zero_()
    Q.attn_o(q, k, v, qn, kn, pos, kc2, vc2, lo.weight, h2, ssq2, att2, scratch, 1e-6, 1e6)
    torch.cuda.synchronize()
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    assert torch.equal(h1, h2), float((h1 - h2).abs().max())
    assert torch.equal(ssq1, ssq2)
    # (beyond one prepare batch att holds o's prepared rows, not the output)


@gpu
@pytest.mark.parametrize("B", [1, 16])
@pytest.mark.parametrize("H,I", [(512, 1024), (4096, 12288)])
def test_linears_fusions(B, H, I):
    # exl3d_linears against the separate ops: RMSNorm prologue (B = 1: in
    # the GEMV's prepare; B = 16: normalized first), residual finish (bit
    # for bit against exl3_matmul, whose launch it is), SwiGLU prologue;
    # at a small shape and at config 4's (hidden 4096, intermediate 12288)
    from plugins_amd import qwen3 as Q
    g = torch.Generator().manual_seed(40 + B + H)
    lq = Q.random_linear(torch, H, H, 4, torch.Generator(device="cuda").manual_seed(1))
    lk = Q.random_linear(torch, H, 256, 4, torch.Generator(device="cuda").manual_seed(2))
    lo = Q.random_linear(torch, H, H, 4, torch.Generator(device="cuda").manual_seed(3))
    ld = Q.random_linear(torch, I, H, 4, torch.Generator(device="cuda").manual_seed(4))
    h = torch.randn(B, H, generator=g)
    w = (1 + 0.1 * torch.randn(H, generator=g)).half()
    hd, ssq = h.cuda(), _ssq(h).cuda()
    # RMSNorm prologue
    yq = torch.empty(B, H, dtype=torch.float16, device="cuda")
    yk = torch.empty(B, 256, dtype=torch.float16, device="cuda")
    Q.linears([lq.weight, lk.weight], hd, outs=[yq, yk], norm_w=w.cuda(), nssq=ssq, eps=1e-6)
    xn = ref_rmsnorm(h, w, 1e-6)
    wq, wk = lq(xn.cuda()).cpu(), lk(xn.cuda()).cpu()
    # the norm's sum in another order moves some f16 inputs by an ulp
    assert rel(yq.cpu(), wq) < 1e-3 and rel(yk.cpu(), wk) < 1e-3
    # residual finish: h += y, and the new sums of squares
    x = torch.randn(B, H, generator=g).half()
    res = hd.clone()
    rssq = torch.empty(B, H // 128, device="cuda")
    Q.linears([lo.weight], x.cuda(), res=res, res_ssq=rssq)
    y = lo(x.cuda()).cpu()
    assert torch.equal(res.cpu(), h + y.float())  # one f32 add of the same y
    assert torch.allclose(rssq.cpu(), _ssq(res.cpu()), rtol=1e-5, atol=0)
    # SwiGLU prologue (B = 16: the SwiGLU first, elementwise)
    gt = torch.randn(B, I, generator=g).half()
    up = torch.randn(B, I, generator=g).half()
    yd = torch.empty(B, H, dtype=torch.float16, device="cuda")
    Q.linears([ld.weight], gt.cuda(), outs=[yd], up=up.cuda())
    hm = (torch.nn.functional.silu(gt.float()) * up.float()).half()
    # the SwiGLU in f32 with expf against torch's: an f16 ulp here and there
    assert rel(yd.cpu(), ld(hm.cuda()).cpu()) < 1e-3


@gpu
@pytest.mark.parametrize("count", [1, 2, 3])
def test_linears_norm_prepare_equals_separate_norm(count):
    # beyond one prepare batch, exl3d_linears forms the RMSNorm and every
    # weight's prepare in one pass (stacked prepared rows); against the norm
    # as its own launch followed by the linears on its output: equal bit for
    # bit (the same norm, the same prepare arithmetic, the same GEMV plan)
    from plugins_amd import qwen3 as Q
    B, H = 16, 4096
    g = torch.Generator().manual_seed(70 + count)
    lins = [Q.random_linear(torch, H, o, 4, torch.Generator(device="cuda").manual_seed(10 + i))
            for i, o in enumerate([4096, 1024, 1024][:count])]
    h = torch.randn(B, H, generator=g).cuda()
    w = (1 + 0.1 * torch.randn(H, generator=g)).half().cuda()
    ssq = _ssq(h.cpu()).cuda()
    outs1 = [torch.empty(B, l.out_features, dtype=torch.float16, device="cuda") for l in lins]
    Q.linears([l.weight for l in lins], h, outs=outs1, norm_w=w, nssq=ssq, eps=1e-6)
    xn = torch.empty(B, H, dtype=torch.float16, device="cuda")
    Q.add_rmsnorm(h.clone(), None, w, xn, 1e-6)
    outs2 = [torch.empty(B, l.out_features, dtype=torch.float16, device="cuda") for l in lins]
    Q.linears([l.weight for l in lins], xn, outs=outs2)
    torch.cuda.synchronize()
    for a, b in zip(outs1, outs2):
        assert torch.equal(a, b), float((a.float() - b.float()).abs().max())


@gpu
def test_silu_mul():
    from plugins_amd import qwen3 as Q
    g = torch.Generator().manual_seed(4)
    a = torch.randn(7, 1000, generator=g).half()
    b = torch.randn(7, 1000, generator=g).half()
    out = torch.empty(7, 1000, dtype=torch.float16, device="cuda")
    Q.silu_mul(a.cuda(), b.cuda(), out)
    want = (torch.nn.functional.silu(a.float()) * b.float()).half()
    assert rel(out.cpu(), want) < 2e-3


def restated_step(m, cfg, batch, kc0, vc0):
    """The decode step in float32 on the CPU (norms, RoPE, KV append,
    attention, SwiGLU, residual adds), its linears the library's EXL3
    matmuls (pinned to the oracle in test_gpu_parity.py); kc0/vc0 are the
    caches as they were before the step appended to them."""
    def lin(L, x):
        return L(x.cuda()).cpu()

    pos, ids = m.pos.cpu(), m.ids.cpu().long()
    h = m.embed_table.cpu()[ids].float()
    add = None
    for li, L in enumerate(m.layers):
        if add is not None:
            h = h + add.float()
        xn = ref_rmsnorm(h, L["in_norm"].cpu(), cfg.eps)
        q, k, v = lin(L["q"], xn), lin(L["k"], xn), lin(L["v"], xn)
        qr = ref_qk_norm_rope(q.view(batch, cfg.heads, 128), L["q_norm"].cpu(), pos, cfg.eps,
                              cfg.theta).view(batch, -1)
        kr = ref_qk_norm_rope(k.view(batch, cfg.kv_heads, 128), L["k_norm"].cpu(), pos, cfg.eps,
                              cfg.theta)
        kc, vc = kc0[li].cpu(), vc0[li].cpu()
        for b in range(batch):
            kc[b, :, int(pos[b])] = kr[b]
            vc[b, :, int(pos[b])] = v[b].view(cfg.kv_heads, 128)
        att = ref_attention(qr, kc, vc, pos)
        o = lin(L["o"], att)
        h = h + o.float()
        xn = ref_rmsnorm(h, L["post_norm"].cpu(), cfg.eps)
        gg, uu = lin(L["gate"], xn), lin(L["up"], xn)
        hm = (torch.nn.functional.silu(gg.float()) * uu.float()).half()
        add = lin(L["down"], hm)
    h = h + add.float()
    return lin(m.lm_head, ref_rmsnorm(h, m.final_norm.cpu(), cfg.eps))


def _step_and_restate(cfg, batch, ctx, seed):
    from plugins_amd import qwen3 as Q
    m = Q.Qwen3Decoder(cfg, batch, ctx, seed=seed)
    m.ids.copy_(torch.randint(0, cfg.vocab, (batch,), dtype=torch.int32,
                              generator=torch.Generator().manual_seed(seed)))
    m.pos.copy_(torch.tensor([ctx - 7 * b for b in range(batch)], dtype=torch.int32))
    kc0 = [L["kc"].clone() for L in m.layers]
    vc0 = [L["vc"].clone() for L in m.layers]
    logits = m.step().cpu()
    torch.cuda.synchronize()
    return m, logits, restated_step(m, cfg, batch, kc0, vc0)


@gpu
@pytest.mark.parametrize("batch", [1, 4])
def test_decode_step_against_float32_restatement(batch):
    from plugins_amd import qwen3 as Q
    cfg = Q.Qwen3Config(layers=2, hidden=1024, heads=8, kv_heads=2, inter=2048, vocab=1024)
    _, logits, want = _step_and_restate(cfg, batch, 300, 5)
    # f16 rounding differences at each op propagate through two layers:
    # 1e-2 relative Frobenius on the logits
    assert rel(logits, want) < 1e-2, rel(logits, want)
    assert torch.isfinite(logits).all()


@gpu
@pytest.mark.parametrize("batch", [1, 16])
def test_decode_step_full_qwen3_8b(batch):
    """BASELINE config 4 at its real shape: 36 layers, hidden 4096, 32/8
    heads, intermediate 12288, vocab 151936, K=4, caches at context 2048;
    the step against the float32 restatement, and its HIP-graph replay
    against the eager step bit for bit (the step is idempotent: it rewrites
    the same cache rows from the same inputs)."""
    from plugins_amd import qwen3 as Q
    cfg = Q.Qwen3Config()
    m, logits, want = _step_and_restate(cfg, batch, 2048, 7 + batch)
    r = rel(logits, want)
    print(f"config 4 batch {batch}: logits rel err {r:.2e}")
    # f16 rounding differences at each op (the fused norms' sums in another
    # order, the attention's online softmax) propagate through 36 layers:
    # 2e-2 relative Frobenius on the logits
    assert r < 2e-2, r
    assert torch.isfinite(logits).all()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        eager = m.step(stream=cap).clone()
    torch.cuda.synchronize()
    assert torch.equal(eager.cpu(), logits)  # repeated eager steps agree
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap, capture_error_mode="thread_local"):
        m.step(stream=cap)
    for _ in range(3):
        m.logits.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(m.logits.cpu(), logits)
