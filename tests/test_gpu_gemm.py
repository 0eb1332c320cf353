"""The split-bf16 fp32 GEMM (e2v2_gemm_s3) against float64 products and against
the native fp32 GEMM of the same operands (torch.mm on the GPU: hipBLASLt on fp32
MFMA).

Error measure: |C - C64| elementwise over the GEMM's own scale sum_k |a_ik| |b_kj|
(the quantity fp32 rounding error is proportional to).  The bar: the maximum of
that measure within 2x of the native fp32 GEMM's on the same operands, and below
8 units of fp32 rounding (2^-24) times sqrt(k)."""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


def _scaled_err(c, a64, w64, res64=None, bias64=None):
    ref = a64 @ w64.transpose(-1, -2)
    scale = a64.abs() @ w64.abs().transpose(-1, -2)
    if bias64 is not None:
        ref = ref + bias64
        scale = scale + bias64.abs()
    if res64 is not None:
        ref = ref + res64
        scale = scale + res64.abs()
    return float(((c.double().cpu() - ref).abs() / (scale + 1e-300)).max())


def _wide_range(shape, gen, spread=8.0):
    """Random values with magnitudes over 2^-spread .. 2^spread and both signs."""
    mag = torch.exp2((torch.rand(shape, generator=gen) * 2 - 1) * spread)
    return (torch.randn(shape, generator=gen).sign() * mag).float()


@pytest.mark.parametrize("m,n,k,batch", [(1000, 256, 256, 9), (130, 128, 32, 1), (1, 768, 1536, 1),
                                         (2048, 512, 768, 3), (517, 1024, 512, 1)])
def test_split_gemm_against_float64_and_native_fp32(pkg, cuda, m, n, k, batch):
    from ubio_molfm_amd import gemm
    g = torch.Generator().manual_seed(m + n + k)
    n_w = min(batch, 3)
    a = torch.randn(batch, m, k, generator=g)
    w = torch.randn(n_w, n, k, generator=g) / math.sqrt(k)
    widx = [b % n_w for b in range(batch)]
    pw = gemm.pack(w.to(cuda))
    out = torch.empty(batch, m, n, device=cuda)
    gemm.gemm(a.to(cuda), pw, out, widx)
    wb = w[widx].double()
    err = _scaled_err(out, a.double(), wb)
    native = torch.stack([a[b].to(cuda) @ w[widx[b]].to(cuda).t() for b in range(batch)])
    err_native = _scaled_err(native, a.double(), wb)
    print(f"m={m} n={n} k={k} batch={batch}: split {err / U:.2f} u, native fp32 {err_native / U:.2f} u")
    assert err <= max(2.0 * err_native, 2 * U) and err <= 8 * U * math.sqrt(k), (err / U, err_native / U)


def test_split_gemm_wide_range_bias_residual_strides(pkg, cuda):
    """Operands over 2^-8..2^8 (every piece matters), a bias on the first batch
    only, the residual read from the output buffer itself, rows of A strided
    (a column slice of a wider matrix) and the weight packed from its transpose."""
    from ubio_molfm_amd import gemm
    g = torch.Generator().manual_seed(7)
    batch, m, n, k = 3, 300, 256, 512
    a_wide = _wide_range((batch, m, k + 64), g)
    a = a_wide[:, :, 32:32 + k]
    wt = _wide_range((2, k, n), g) / k            # packed transposed: W_w = wt[w]^T
    bias = _wide_range((n,), g)
    res = _wide_range((batch, m, n), g)
    widx = [1, 0, 1]
    pw = gemm.pack(wt.to(cuda), transpose=True)
    a_dev = a_wide.to(cuda)[:, :, 32:32 + k]
    assert a_dev.stride(1) == k + 64
    out = res.to(cuda).clone()
    gemm.gemm(a_dev, pw, out, widx, bias=bias.to(cuda), bias_batches=1, res=out)
    w64 = wt[widx].double().transpose(1, 2)
    b64 = torch.zeros(batch, 1, n, dtype=torch.float64)
    b64[0, 0] = bias.double()
    err = _scaled_err(out, a.double(), w64, res64=res.double(), bias64=b64)
    print(f"wide range: {err / U:.2f} u")
    assert err <= 8 * U * math.sqrt(k)


def test_split_gemm_exact_on_representable_products(pkg, cuda):
    """Integer operands whose products and sums are exact in fp32: the split
    GEMM must return them exactly (any dropped piece product or wrong piece
    pairing shows as an integer error)."""
    from ubio_molfm_amd import gemm
    g = torch.Generator().manual_seed(3)
    m, n, k = 257, 128, 64
    a = torch.randint(-2 ** 11, 2 ** 11, (m, k), generator=g).float()      # 12-bit: needs two bf16 pieces
    w = torch.randint(-2 ** 5, 2 ** 5, (n, k), generator=g).float()
    pw = gemm.pack(w.to(cuda))
    out = torch.empty(m, n, device=cuda)
    gemm.gemm(a.to(cuda), pw, out)
    ref = (a.double() @ w.double().t())
    assert ref.abs().max() < 2 ** 24
    assert torch.equal(out.cpu().double(), ref)


def test_split_gemm_rejects_bad_shapes(pkg, cuda):
    from ubio_molfm_amd import gemm
    with pytest.raises(ValueError):
        gemm.pack(torch.randn(100, 64, device=cuda))              # n not a multiple of 128
    pw = gemm.pack(torch.randn(128, 64, device=cuda))
    with pytest.raises(ValueError):
        gemm.gemm(torch.randn(10, 32, device=cuda), pw, torch.empty(10, 128, device=cuda))
    out = torch.empty(0, 128, device=cuda)
    gemm.gemm(torch.empty(0, 64, device=cuda), pw, out)            # no rows: nothing to do


@pytest.mark.parametrize("n,with_v,with_bias", [(1, True, True), (300, False, True), (1000, True, False)])
def test_qk_proj_split(pkg, cuda, n, with_v, with_bias):
    """Split-GEMM Q/K projection + m-contraction (forward) and its input gradient
    with the value projection's gradient folded in (backward) against float64, at
    the fp32 fused kernel's tolerances (2e-5 forward, 1e-4 gradient)."""
    from ubio_molfm_amd import gemm
    torch.manual_seed(7)
    hid, C, Cv = 512, 256, 256
    print(f"[qk_proj s3] n={n} with_v={with_v} bias={with_bias}", flush=True)
    idx = torch.tensor([0, 1, 1, 1, 2, 2, 2, 2, 2], device=cuda)
    x = torch.randn(9, n, C, device=cuda)
    W = torch.randn(3, 4 * hid, C, device=cuda) / 16
    bias = torch.randn(4 * hid, device=cuda) if with_bias else None
    Wv = torch.randn(3, Cv, C, device=cuda) / 16
    P = gemm.pack_qk(W, bias, Wv)
    hq, hk, y = gemm.qk_forward(x, P)
    _, bwd_order = gemm.qk_orders(hid)
    y_model = torch.empty_like(y)
    y_model[:, :, torch.as_tensor(bwd_order, device=cuda)] = y        # back to W's column order
    L = [slice(0, 1), slice(1, 4), slice(4, 9)]
    xd = x.double().requires_grad_(True)
    yd = torch.bmm(xd, W.double()[idx].transpose(1, 2))
    if with_bias:
        shift = torch.zeros(9, 1, 4 * hid, device=cuda, dtype=torch.float64)
        shift[0, 0] = bias.double()
        yd = yd + shift
    aq, bq, ak, bk = yd.split(hid, dim=2)
    hqd = torch.cat([(aq[s] * bq[s]).sum(0) for s in L], dim=1)
    hkd = torch.cat([(ak[s] * bk[s]).sum(0) for s in L], dim=1)
    rel = lambda a, b: float((a.double() - b).norm() / (b.norm() + 1e-30))
    e_y, e_q, e_k = rel(y_model, yd.detach()), rel(hq, hqd.detach()), rel(hk, hkd.detach())
    ghq = torch.randn(n, 3 * hid, device=cuda); ghk = torch.randn(n, 3 * hid, device=cuda)
    gv = torch.randn(9, n, Cv, device=cuda) if with_v else None
    gx = gemm.qk_backward(y, ghq, ghk, gv, P)
    obj = (hqd * ghq.double()).sum() + (hkd * ghk.double()).sum()
    if with_v:
        obj = obj + (torch.bmm(xd, Wv.double()[idx].transpose(1, 2)) * gv.double()).sum()
    gxd, = torch.autograd.grad(obj, xd)
    e_g = rel(gx, gxd)
    print(f"[qk_proj s3] n={n} y {e_y:.2e} hq {e_q:.2e} hk {e_k:.2e} gx {e_g:.2e}", flush=True)
    assert e_y < 2e-5 and e_q < 2e-5 and e_k < 2e-5
    assert e_g < 1e-4


@pytest.mark.parametrize("n", [1, 700])
def test_qk_heads_batched_split(pkg, cuda, n):
    """The query and key final_linear stacks (Linear 1536->512, LayerNorm, SiLU,
    Linear 512->1024) run as two-batch split GEMMs: outputs and input gradients
    against the two stacks evaluated separately in float64."""
    import copy
    from ubio_molfm_amd import modules
    torch.manual_seed(11)
    print(f"[qk heads s3] n={n}", flush=True)
    mk = lambda: torch.nn.Sequential(torch.nn.Linear(1536, 512), torch.nn.LayerNorm(512), torch.nn.SiLU(),
                                     torch.nn.Linear(512, 1024))
    fq, fk = mk(), mk()
    with torch.no_grad():                      # LayerNorm affine away from its (1, 0) init
        for f in (fq, fk):
            f[1].weight.uniform_(0.5, 1.5)
            f[1].bias.uniform_(-0.5, 0.5)
    fq, fk = fq.to(cuda), fk.to(cuda)
    P = modules.head_pair_packs(fq, fk, fq)
    assert P is not None
    hq = torch.randn(n, 1536, device=cuda, requires_grad=True)
    hk = torch.randn(n, 1536, device=cuda, requires_grad=True)
    q, k = modules.QKHeadsS3Fn.apply(hq, hk, P)
    gq, gk = torch.randn_like(q), torch.randn_like(k)
    gxq, gxk = torch.autograd.grad((q * gq).sum() + (k * gk).sum(), (hq, hk))
    fqd, fkd = copy.deepcopy(fq).double(), copy.deepcopy(fk).double()
    hqd = hq.detach().double().requires_grad_(True)
    hkd = hk.detach().double().requires_grad_(True)
    qd, kd = fqd(hqd), fkd(hkd)
    gqd, gkd = torch.autograd.grad((qd * gq.double()).sum() + (kd * gk.double()).sum(), (hqd, hkd))
    rel = lambda a, b: float((a.double() - b).norm() / (b.norm() + 1e-30))
    errs = [rel(q, qd.detach()), rel(k, kd.detach()), rel(gxq, gqd), rel(gxk, gkd)]
    print(f"[qk heads s3] n={n} q {errs[0]:.2e} k {errs[1]:.2e} gq {errs[2]:.2e} gk {errs[3]:.2e}", flush=True)
    assert max(errs[:2]) < 2e-6 and max(errs[2:]) < 1e-5


def test_grouped_gemm_matches_separate_launches(pkg, cuda):
    """Three GEMMs of different m, n, k (one with a bias, one with a residual read
    from its output, one batched) in one grouped launch: bitwise equal to three
    separate launches (the same per-tile arithmetic), and every group written."""
    from ubio_molfm_amd import gemm
    g = torch.Generator().manual_seed(5)
    specs = [(3000, 256, 768, 1), (1000, 128, 256, 1), (517, 384, 512, 2)]
    probs, refs = [], []
    for i, (m, n, k, batch) in enumerate(specs):
        a = torch.randn(batch, m, k, generator=g).to(cuda)
        pw = gemm.pack((torch.randn(1, n, k, generator=g) / math.sqrt(k)).to(cuda))
        bias = torch.randn(n, generator=g).to(cuda) if i == 0 else None
        res = torch.randn(batch, m, n, generator=g).to(cuda) if i == 1 else None
        widx = [0] * batch
        ref = torch.empty(batch, m, n, device=cuda) if res is None else res.clone()
        gemm.gemm(a, pw, ref, widx, bias=bias, res=None if res is None else ref)
        out = torch.full((batch, m, n), float("nan"), device=cuda) if res is None else res.clone()
        probs.append({"a": a, "pw": pw, "out": out, "widx": widx, "bias": bias, "res": None if res is None else out})
        refs.append(ref)
    gemm.gemm_grouped(probs)
    for p, ref in zip(probs, refs):
        assert torch.equal(p["out"], ref)


@pytest.mark.parametrize("n", [1, 1000])
def test_gated_gemm_equals_gate_kernel_then_gemm(pkg, cuda, n):
    """The FFN's gate applied inside the split GEMM's operand read
    (e2v2_gemm_s3_gated) against the gate kernel (e2v2_gate_fwd) followed by the
    plain split GEMM: the same products, so the outputs are bitwise equal; a
    bias on row 0 and a residual included."""
    from ubio_molfm_amd import _lib, gemm, modules
    g = torch.Generator().manual_seed(9)
    C = 256
    h = torch.randn(9, n, C, generator=g).to(cuda)
    sc = (2 * torch.randn(n, 3 * C, generator=g)).to(cuda)
    w = (torch.randn(3, C, C, generator=g) / 16).to(cuda)
    b2 = torch.randn(C, generator=g).to(cuda)
    res = torch.randn(9, n, C, generator=g).to(cuda)
    widx = [0, 1, 1, 1, 2, 2, 2, 2, 2]
    pw = gemm.pack(w)
    y = torch.empty_like(h)
    k1, k2 = modules.SILU_NORM, modules.SIGMOID_NORM
    _lib.call("e2v2_gate_fwd", _lib.vp(sc.data_ptr()), _lib.vp(h.data_ptr()), _lib.vp(y.data_ptr()), _lib.i32(n),
              _lib.f32(k1), _lib.f32(k2), _lib.vp(torch.cuda.current_stream().cuda_stream))
    ref = torch.empty(9, n, C, device=cuda)
    gemm.gemm(y, pw, ref, widx, bias=b2, res=res)
    out = torch.empty(9, n, C, device=cuda)
    gemm.gemm(h, pw, out, widx, bias=b2, res=res, gate=(sc, k1, k2))
    assert torch.equal(out, ref)


def test_list_operands_either_order(pkg, cuda):
    """Two separately allocated matrices as a two-batch A operand (batch stride =
    their address difference, of either sign, per-batch bias): bitwise equal to
    two single launches."""
    from ubio_molfm_amd import gemm
    g = torch.Generator().manual_seed(13)
    m, n, k = 700, 256, 512
    x0 = torch.randn(m, k, generator=g).to(cuda)
    x1 = torch.randn(m, k, generator=g).to(cuda)
    w = (torch.randn(2, n, k, generator=g) / math.sqrt(k)).to(cuda)
    bias = torch.randn(2, n, generator=g).to(cuda)
    pw = gemm.pack(w)
    refs = []
    for b, x in enumerate((x0, x1)):
        r = torch.empty(m, n, device=cuda)
        gemm.gemm(x, pw, r, [b], bias=bias[b].contiguous())
        refs.append(r)
    for order in ((0, 1), (1, 0)):
        xs = [(x0, x1)[i] for i in order]
        out = torch.empty(2, m, n, device=cuda)
        gemm.gemm(xs, pw, out, list(order), bias=bias[list(order)].contiguous(), bias_batches=2)
        assert torch.equal(out[0], refs[order[0]]) and torch.equal(out[1], refs[order[1]])


# --------------------------------------------------------------------------- one-piece packs: the bf16 mode

def _bf(t):
    return t.to(torch.bfloat16).double()


@pytest.mark.parametrize("a_dtype,c_dtype", [(torch.float32, torch.float32), (torch.bfloat16, torch.float32),
                                             (torch.float32, torch.bfloat16), (torch.bfloat16, torch.bfloat16)])
def test_bf16_gemm_against_float64_on_rounded_operands(pkg, cuda, a_dtype, c_dtype):
    """One-piece packs (the bf16 mode's GEMMs: bf16 operands, fp32 accumulation):
    A read as fp32 and rounded to bf16 as the kernel reads it, or read as bf16;
    the result against the float64 product of the bf16-rounded operands, within
    fp32 accumulation error (8 u sqrt(k) of the GEMM's own scale), plus one bf16
    rounding when C is written as bf16.  A bias on batch 0, a residual and three
    weights over five batches."""
    from ubio_molfm_amd import gemm
    g = torch.Generator().manual_seed(11)
    batch, m, n, k = 5, 333, 256, 768
    a = _wide_range((batch, m, k), g, spread=4.0)
    w = _wide_range((3, n, k), g, spread=4.0) / k
    bias = torch.randn(n, generator=g)
    widx = [0, 1, 2, 1, 0]
    pw = gemm.pack(w.to(cuda), pieces=1)
    assert pw.pieces == 1
    out = torch.empty(batch, m, n, device=cuda, dtype=c_dtype)
    res = None
    if c_dtype == torch.float32:
        res = torch.randn(batch, m, n, generator=g)
        out.copy_(res.to(cuda))
    gemm.gemm(a.to(cuda).to(a_dtype), pw, out, widx, bias=bias.to(cuda), bias_batches=1,
              res=None if res is None else out)
    a64, w64 = _bf(a), _bf(w[widx])
    b64 = torch.zeros(batch, 1, n, dtype=torch.float64)
    b64[0, 0] = bias.double()
    err = _scaled_err(out.float(), a64, w64, res64=None if res is None else res.double(), bias64=b64)
    tol = 8 * U * math.sqrt(k) + (2.0 ** -8 if c_dtype == torch.bfloat16 else 0.0)
    print(f"[bf16 gemm] A {a_dtype} C {c_dtype}: {err / U:.2f} u (tol {tol / U:.0f} u)", flush=True)
    assert err <= tol
    # exactly one product: the second and third pieces of either operand must not enter
    ex = _scaled_err(out.float(), a.double(), w[widx].double(), res64=None if res is None else res.double(),
                     bias64=b64)
    assert ex > 8 * U * math.sqrt(k)


def test_bf16_gemm_gated_and_grouped_match_separate_launches(pkg, cuda):
    """The gated and the grouped forms on one-piece packs equal, bitwise, the gate
    kernel followed by the plain GEMM and the separate launches of the same
    problems (the same products in the same order)."""
    from ubio_molfm_amd import gemm, modules, _lib
    g = torch.Generator().manual_seed(12)
    n_rows, C = 700, 256
    h = torch.randn(9, n_rows, C, generator=g).to(cuda)
    sc = torch.randn(n_rows, 3 * C, generator=g).to(cuda)
    w2 = (torch.randn(3, C, C, generator=g) / 16).to(cuda)
    pw = gemm.pack(w2, pieces=1)
    widx = modules._m_degrees(2)
    k1, k2 = modules.SILU_NORM, modules.SIGMOID_NORM
    y_g = torch.empty(9, n_rows, C, device=cuda)
    gemm.gemm(h, pw, y_g, widx, gate=(sc, k1, k2))
    gated = torch.empty_like(h)
    _lib.call("e2v2_gate_fwd", _lib.vp(sc.data_ptr()), _lib.vp(h.data_ptr()), _lib.vp(gated.data_ptr()),
              _lib.i32(n_rows), _lib.f32(k1), _lib.f32(k2), _lib.vp(torch.cuda.current_stream().cuda_stream))
    y_s = torch.empty_like(y_g)
    gemm.gemm(gated, pw, y_s, widx)
    assert torch.equal(y_g, y_s)
    a1 = torch.randn(2, 300, 512, generator=g).to(cuda).to(torch.bfloat16)
    a2 = torch.randn(3, 500, 256, generator=g).to(cuda).to(torch.bfloat16)
    p1 = gemm.pack((torch.randn(2, 256, 512, generator=g) / 16).to(cuda), pieces=1)
    p2 = gemm.pack((torch.randn(1, 384, 256, generator=g) / 16).to(cuda), pieces=1)
    o1 = torch.empty(2, 300, 256, device=cuda)
    o2 = torch.empty(3, 500, 384, device=cuda, dtype=torch.bfloat16)
    gemm.gemm_grouped([{"a": a1, "pw": p1, "out": o1}, {"a": a2, "pw": p2, "out": o2, "widx": [0, 0, 0]}])
    r1, r2 = torch.empty_like(o1), torch.empty_like(o2)
    gemm.gemm(a1, p1, r1)
    gemm.gemm(a2, p2, r2, [0, 0, 0])
    assert torch.equal(o1, r1) and torch.equal(o2, r2)
    with pytest.raises(ValueError):                                   # a bf16 A needs a one-piece packing
        gemm.gemm(a1[0], gemm.pack((torch.randn(256, 512, generator=g)).to(cuda)), o1[0])


def test_qk_proj_one_piece_against_float64(pkg, cuda):
    """The Q/K projection kernels on one-piece packs: forward against float64 of
    the bf16-rounded weights and input (the input rounded in the kernel), at
    fp32 accumulation error."""
    from ubio_molfm_amd import gemm
    torch.manual_seed(9)
    n, hid, C, Cv = 300, 512, 256, 256
    W = torch.randn(3, 4 * hid, C, device=cuda) / 16
    b = torch.randn(4 * hid, device=cuda)
    Wv = torch.randn(3, Cv, C, device=cuda) / 16
    P = gemm.pack_qk(W, b, Wv, pieces=1)
    x = torch.randn(9, n, C, device=cuda)
    hq, hk, _ = gemm.qk_forward(x, P)
    idx = torch.tensor([0, 1, 1, 1, 2, 2, 2, 2, 2])
    x64, W64 = _bf(x.cpu()), _bf(W.cpu())
    y = torch.einsum("mnc,moc->mno", x64, W64[idx])
    y[0] += b.cpu().double()
    ref = [torch.stack([(y[a:c, :, o0:o0 + hid] * y[a:c, :, o1:o1 + hid]).sum(0)
                        for (a, c) in ((0, 1), (1, 4), (4, 9))], 1).reshape(n, 3 * hid)
           for (o0, o1) in ((0, hid), (2 * hid, 3 * hid))]
    for got, r in zip((hq, hk), ref):
        rel = float((got.cpu().double() - r).norm() / r.norm())
        print(f"[qk one-piece] rel {rel:.2e}", flush=True)
        assert rel < 2e-5


def test_qk_proj_one_piece_bf16_y_backward(pkg, cuda):
    """One-piece packs keep y as bf16 (the bf16 mode): y within one bf16 rounding
    of the float64 product, hq / hk from the fp32 sums as before, and the input
    gradient equal, at fp32 accumulation error, to float64 GEMMs of exactly the
    operands the kernel forms: the contraction gradient g * y(partner) from the
    stored bf16 y, multiplied in fp32 and rounded to bf16, the value gradient
    and both weights rounded to bf16."""
    from ubio_molfm_amd import gemm
    torch.manual_seed(10)
    n, hid, C, Cv = 300, 512, 256, 256
    W = torch.randn(3, 4 * hid, C, device=cuda) / 16
    b = torch.randn(4 * hid, device=cuda)
    Wv = torch.randn(3, Cv, C, device=cuda) / 16
    P = gemm.pack_qk(W, b, Wv, pieces=1)
    x = torch.randn(9, n, C, device=cuda)
    hq, hk, y = gemm.qk_forward(x, P)
    assert y.dtype == torch.bfloat16
    hq32, hk32, y32 = gemm.qk_forward(x, P, y_bf16=False)
    assert torch.equal(hq, hq32) and torch.equal(hk, hk32) and torch.equal(y, y32.to(torch.bfloat16))
    _, bwd_order = gemm.qk_orders(hid)
    ym = torch.empty(9, n, 4 * hid, dtype=torch.float32, device=cuda)
    ym[:, :, torch.as_tensor(bwd_order, device=cuda)] = y.float()      # W's column order
    idx = torch.tensor([0, 1, 1, 1, 2, 2, 2, 2, 2])
    yd = torch.einsum("mnc,moc->mno", _bf(x.cpu()), _bf(W.cpu())[idx])
    yd[0] += b.cpu().double()
    assert float((ym.cpu().double() - yd).abs().max() / yd.abs().max()) < 4e-3
    ghq = torch.randn(n, 3 * hid, device=cuda); ghk = torch.randn(n, 3 * hid, device=cuda)
    gv = torch.randn(9, n, Cv, device=cuda)
    gx = gemm.qk_backward(y, ghq, ghk, gv, P)
    lm = [0, 1, 1, 1, 2, 2, 2, 2, 2]
    gy = torch.empty(9, n, 4 * hid, dtype=torch.float32)
    yc = ym.cpu()
    for m in range(9):
        l = lm[m]
        gq, gk = ghq.cpu()[:, l * hid:(l + 1) * hid], ghk.cpu()[:, l * hid:(l + 1) * hid]
        qa, qb, ka, kb = yc[m].split(hid, dim=1)
        gy[m] = torch.cat([qb * gq, qa * gq, kb * gk, ka * gk], dim=1)     # fp32 products, as the kernel forms them
    gy = gy.to(torch.bfloat16).double()
    ref = torch.einsum("mno,mok->mnk", gy, _bf(W.cpu())[idx]) + \
        torch.einsum("mnj,mjk->mnk", _bf(gv.cpu()), _bf(Wv.cpu())[idx])
    rel = float((gx.cpu().double() - ref).norm() / ref.norm())
    print(f"[qk one-piece bf16 y] gx rel {rel:.2e}", flush=True)
    assert rel < 2e-5
