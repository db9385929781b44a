"""Parity of the HIP LayerAdam step (through the C-ABI) with the CPU checker.

Bar: fp32 p/m/v and 16-bit states bit-exact against the oracle (which is
itself bit-exact against the reference compiled from its sources, see
test_oracle.py); the bf16 compute copy bit-exact to RNE of the updated fp32
master; the grad norm within 1e-12 relative of the oracle's compensated
float64 sum, which is the exact sum to about one binary64 ulp (the tolerance
north_star allows is 1e-6); NaN compared as a class.
"""
from __future__ import annotations

import zlib

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests import _golden as G
from tests import _hip as H

pytestmark = pytest.mark.gpu

KIND16 = {"bf16": "bf16", "f16": "f16", "f32": None}


def _view(bits_arr, kind):
    return bits_arr.view(np.float32) if kind == "f32" else bits_arr


def log(msg):
    print(msg, flush=True)


# ---------------------------------------------------------------------------
# golden fixtures written by the compiled reference
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name", G.case_names())
def test_hip_reproduces_golden(name, hip_device):
    log(f"golden case {name}")
    meta, arrays = G.get_case(name)
    pk, gk, sk = meta["triple"]
    b1, b2 = meta["betas"]
    opt = H.HipAdam(1e-3, (b1, b2), meta["eps"], meta["wd"], meta["adamw"])
    dev = {}

    def call(step, lr, p, g, m, v, lo, hi):
        # keep the state resident; upload the step's grads once per step
        if "p" not in dev:
            dev["p"] = H.to_dev_bits(p, pk, hip_device)
            dev["m"] = H.to_dev_bits(m, sk, hip_device)
            dev["v"] = H.to_dev_bits(v, sk, hip_device)
        if dev.get("gstep") != step:
            dev["g"] = H.to_dev_bits(g, gk, hip_device)
            dev["gstep"] = step
        opt.update(step, lr, b1, b2, meta["eps"], meta["wd"], meta["bc"], dev["p"][lo:hi],
                   dev["g"][lo:hi], dev["m"][lo:hi], dev["v"][lo:hi])
        if hi == sum(meta["sizes"]):
            p[:] = H.to_np_bits(dev["p"], pk)
            m[:] = H.to_np_bits(dev["m"], sk)
            v[:] = H.to_np_bits(dev["v"], sk)

    got = G.replay(meta, arrays, call)
    assert G.mismatches(meta, arrays, got) == (0, 0, 0)


# ---------------------------------------------------------------------------
# config C1: one GPT-2-small block, 10 steps, bf16 copy emitted
# ---------------------------------------------------------------------------

GPT2_SIZES = [768, 768, 768 * 2304, 2304, 768 * 768, 768, 768, 768, 768 * 3072, 3072, 3072 * 768, 768]


def test_c1_gpt2_block_ten_steps(hip_device):
    from slideformer_amd import LayerAdam
    n = sum(GPT2_SIZES)
    assert n == 7_087_872
    log(f"C1 n={n}")
    rng = np.random.default_rng(1)
    p_host = rng.normal(0, 0.02, n).astype(np.float32)
    m_host = np.zeros(n, np.float32)
    v_host = np.zeros(n, np.float32)
    orc = O.OracleAdam(1e-5, (0.9, 0.999), 1e-8, 0.01, True)

    opt = LayerAdam(lr=1e-5, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    p_dev = torch.from_numpy(p_host.copy()).to(hip_device)
    params = [torch.nn.Parameter(t) for t in torch.split(p_dev, GPT2_SIZES)]
    idx = opt.add_layer_params(0, params)
    assert idx == 0 and opt.exp_avg_flat[0].device == p_dev.device
    out = torch.empty(n, dtype=torch.bfloat16, device=hip_device)
    for step in range(1, 11):
        g32 = np.random.default_rng(1000 + step).normal(0, 1e-3, n).astype(np.float32)
        g_bf = torch.from_numpy(g32).bfloat16()
        g_bits = H.to_np_bits(g_bf, "bf16")
        group = opt.begin_chunk_step(0)
        opt.step_chunk(p_dev, g_bf.to(hip_device), opt.exp_avg_flat[0], opt.exp_avg_sq_flat[0], group,
                       bf16_out=out)
        opt.end_chunk_step(0)
        orc.update(step, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, p_host, g_bits, m_host, v_host, g16="bf16")
    torch.cuda.synchronize()
    assert np.array_equal(H.to_np_bits(p_dev, "f32"), p_host.view(np.uint32))
    assert np.array_equal(H.to_np_bits(opt.exp_avg_flat[0], "f32"), m_host.view(np.uint32))
    assert np.array_equal(H.to_np_bits(opt.exp_avg_sq_flat[0], "f32"), v_host.view(np.uint32))
    assert np.array_equal(H.to_np_bits(out, "bf16"), O.f32_to_bf16(p_host))
    # the per-param views see the flat buffer (layer_adam.py:176-189)
    assert torch.equal(params[2].data, p_dev[1536:1536 + 768 * 2304])


# ---------------------------------------------------------------------------
# tails, misaligned sub-views, every dtype triple
# ---------------------------------------------------------------------------

SIZES = [1, 3, 7, 8, 15, 16, 17, 31, 63, 64, 127, 129, 1023, 4097, 100_003]


@pytest.mark.parametrize("offsets", [(0, 0, 0, 0), (1, 1, 1, 1), (3, 3, 3, 3), (5, 5, 5, 5),
                                     (0, 1, 0, 0), (2, 0, 4, 6), (7, 3, 1, 0)])
def test_sizes_and_misaligned_offsets(offsets, hip_device):
    op, og, om, ov = offsets
    log(f"offsets {offsets}")
    rng = np.random.default_rng(sum(offsets) * 31 + op)
    opt = H.HipAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    total = sum(SIZES)
    P = torch.from_numpy(rng.normal(0, 0.02, total + 8).astype(np.float32)).to(hip_device)
    M = torch.from_numpy(rng.normal(0, 1e-3, total + 8).astype(np.float32)).to(hip_device)
    V = torch.from_numpy(np.abs(rng.normal(0, 1e-6, total + 8)).astype(np.float32)).to(hip_device)
    OUT = torch.zeros(total + 8, dtype=torch.bfloat16, device=hip_device)
    ph, mh, vh = H.to_np_bits(P, "f32"), H.to_np_bits(M, "f32"), H.to_np_bits(V, "f32")
    for step in (1, 2):
        gb = torch.from_numpy(rng.normal(0, 1e-3, total + 8).astype(np.float32)).bfloat16()
        G_ = gb.to(hip_device)
        gh = H.to_np_bits(gb, "bf16")
        lo = 0
        for n in SIZES:
            opt.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, P[op + lo:op + lo + n],
                       G_[og + lo:og + lo + n], M[om + lo:om + lo + n], V[ov + lo:ov + lo + n],
                       out=OUT[op + lo:op + lo + n])
            orc.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, ph.view(np.float32)[op + lo:op + lo + n],
                       gh[og + lo:og + lo + n], mh.view(np.float32)[om + lo:om + lo + n],
                       vh.view(np.float32)[ov + lo:ov + lo + n], g16="bf16")
            lo += n
    torch.cuda.synchronize()
    assert np.array_equal(H.to_np_bits(P, "f32"), ph)
    assert np.array_equal(H.to_np_bits(M, "f32"), mh)
    assert np.array_equal(H.to_np_bits(V, "f32"), vh)
    out = H.to_np_bits(OUT, "bf16")
    seg = slice(op, op + total)
    assert np.array_equal(out[seg], O.f32_to_bf16(ph.view(np.float32)[seg]))


TRIPLES = [("f32", "bf16", "f32"), ("f32", "f32", "f32"), ("f32", "f16", "f32"),
           ("bf16", "bf16", "f32"), ("bf16", "f32", "f32"), ("bf16", "bf16", "bf16"),
           ("f16", "f16", "f32"), ("f16", "f32", "f32"), ("f16", "f16", "f16")]


@pytest.mark.parametrize("triple", TRIPLES)
@pytest.mark.parametrize("mode", ["adamw", "l2", "none", "no_bc"])
def test_every_triple_and_mode(triple, mode, hip_device):
    pk, gk, sk = triple
    log(f"triple {triple} mode {mode}")
    wd = 0.0 if mode == "none" else 0.05
    adamw = mode != "l2"
    bc = mode != "no_bc"
    rng = np.random.default_rng(zlib.crc32(repr((triple, mode)).encode()))
    sizes = (100_003, 4096, 13)
    n = sum(sizes)
    p = torch.from_numpy(rng.normal(0, 0.02, n).astype(np.float32)).to(H.TD[pk])
    m = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).to(H.TD[sk])
    v = torch.from_numpy(np.abs(rng.normal(0, 1e-6, n)).astype(np.float32)).to(H.TD[sk])
    ph, mh, vh = H.to_np_bits(p, pk), H.to_np_bits(m, sk), H.to_np_bits(v, sk)
    pd, md, vd = p.to(hip_device), m.to(hip_device), v.to(hip_device)
    opt = H.HipAdam(1e-3, (0.9, 0.999), 1e-8, wd, adamw)
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, wd, adamw)
    for step in (1, 2, 3):
        g = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).to(H.TD[gk])
        gh = H.to_np_bits(g, gk)
        gd = g.to(hip_device)
        lo = 0
        for size in sizes:
            hi = lo + size
            opt.update(step, 1e-3, 0.9, 0.999, 1e-8, wd, bc, pd[lo:hi], gd[lo:hi], md[lo:hi], vd[lo:hi])
            orc.update(step, 1e-3, 0.9, 0.999, 1e-8, wd, bc, _view(ph, pk)[lo:hi], _view(gh, gk)[lo:hi],
                       _view(mh, sk)[lo:hi], _view(vh, sk)[lo:hi], p16=KIND16[pk], g16=KIND16[gk],
                       s16=KIND16[sk])
            lo = hi
    torch.cuda.synchronize()
    assert G.same_bits(H.to_np_bits(pd, pk), ph, pk).all()
    assert G.same_bits(H.to_np_bits(md, sk), mh, sk).all()
    assert G.same_bits(H.to_np_bits(vd, sk), vh, sk).all()


@pytest.mark.parametrize("kind", ["bf16", "f16"])
@pytest.mark.parametrize("offsets", [(0, 0, 0, 0, 0), (1, 1, 1, 1, 1), (3, 3, 3, 3, 3), (4, 4, 4, 4, 4),
                                     (7, 7, 7, 7, 7), (0, 4, 0, 0, 0), (2, 2, 6, 2, 2), (5, 1, 3, 7, 0)])
def test_all_16bit_triples_every_head_phase(kind, offsets, hip_device):
    """The all-16-bit triples ((bf16, bf16, bf16), (f16, f16, f16)) run a kernel
    whose lanes own 8 consecutive elements: the head that aligns every stream,
    the bf16 copy included, to 8-element (16-byte) groups, the 512-element
    runs, the remainder and the reference's scalar tail.  Every head phase
    0-7, phases that agree only modulo 4 (then the call takes la_adamw_kernel's
    4-element layout), sizes around 8, 16, 512 and the tail, with the bf16 copy and a clip
    coefficient: every bit equals the oracle's."""
    op, og, om, ov, oo = offsets
    log(f"16-bit triple {kind} offsets {offsets}")
    rng = np.random.default_rng(zlib.crc32(repr((kind, offsets)).encode()))
    sizes = (1, 7, 8, 15, 16, 17, 511, 512, 513, 1023, 4099, 70_001, 100_003)
    total = sum(sizes)
    td = H.TD[kind]
    P = torch.from_numpy(rng.normal(0, 0.02, total + 8).astype(np.float32)).to(td).to(hip_device)
    M = torch.from_numpy(rng.normal(0, 1e-3, total + 8).astype(np.float32)).to(td).to(hip_device)
    V = torch.from_numpy(np.abs(rng.normal(0, 1e-6, total + 8)).astype(np.float32)).to(td).to(hip_device)
    OUT = torch.zeros(total + 8, dtype=torch.bfloat16, device=hip_device)
    ph, mh, vh = H.to_np_bits(P, kind), H.to_np_bits(M, kind), H.to_np_bits(V, kind)
    oh = np.zeros(total + 8, np.uint16)
    coef = torch.tensor([0.625], device=hip_device)
    opt = H.HipAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    for step in (1, 2):
        g = torch.from_numpy(rng.normal(0, 1e-3, total + 8).astype(np.float32)).to(td)
        gd, gh = g.to(hip_device), H.to_np_bits(g, kind)
        lo = 0
        for n in sizes:
            opt.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, P[op + lo:op + lo + n], gd[og + lo:og + lo + n],
                       M[om + lo:om + lo + n], V[ov + lo:ov + lo + n], out=OUT[oo + lo:oo + lo + n], coef=coef)
            orc.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, ph[op + lo:op + lo + n], gh[og + lo:og + lo + n],
                       mh[om + lo:om + lo + n], vh[ov + lo:ov + lo + n], p16=kind, g16=kind, s16=kind,
                       p_bf16_out=oh[oo + lo:oo + lo + n], clip_coef=0.625)
            lo += n
    torch.cuda.synchronize()
    assert G.same_bits(H.to_np_bits(P, kind), ph, kind).all()
    assert G.same_bits(H.to_np_bits(M, kind), mh, kind).all()
    assert G.same_bits(H.to_np_bits(V, kind), vh, kind).all()
    assert np.array_equal(H.to_np_bits(OUT, "bf16")[oo:oo + total], oh[oo:oo + total])


def test_denormal_and_extreme_values(hip_device):
    """Subnormal v and grads, zero grads, huge grads: IEEE denormals are kept."""
    log("denormals")
    n = 4096 + 5
    rng = np.random.default_rng(9)
    g = rng.normal(0, 1e-3, n).astype(np.float32)
    g[0::3] = rng.normal(0, 1e-22, g[0::3].size)   # squares underflow into subnormals
    g[1::7] = 0.0
    g[2::11] = rng.normal(0, 1e3, g[2::11].size)
    p = rng.normal(0, 0.02, n).astype(np.float32)
    p[5::13] = 1e-40                                # subnormal params
    m = np.zeros(n, np.float32)
    v = np.full(n, 1e-44, np.float32)               # subnormal second moment
    pd, gd, md, vd = (torch.from_numpy(x.copy()).to(hip_device) for x in (p, g, m, v))
    opt = H.HipAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    for step in (1, 2):
        opt.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, pd, gd, md, vd)
        orc.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, p, g.copy(), m, v)
    torch.cuda.synchronize()
    assert np.array_equal(H.to_np_bits(pd, "f32"), p.view(np.uint32))
    assert np.array_equal(H.to_np_bits(md, "f32"), m.view(np.uint32))
    assert np.array_equal(H.to_np_bits(vd, "f32"), v.view(np.uint32))


# ---------------------------------------------------------------------------
# grad norm + clip
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n", [1, 7, 4097, 1_000_003, 16 * 1024 * 1024 + 5])
@pytest.mark.parametrize("gk", ["bf16", "f32", "f16"])
def test_grad_sqnorm(n, gk, hip_device):
    log(f"sqnorm n={n} {gk}")
    rng = np.random.default_rng(n)
    g = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).to(H.TD[gk])
    gh = H.to_np_bits(g, gk)
    gd = g.to(hip_device)
    sq = H.sqnorm(gd)
    sq2 = H.sqnorm(gd)
    exact = O.grad_sqnorm(_view(gh, gk), KIND16[gk])
    got = float(sq.item())
    assert abs(got - exact) <= 1e-12 * exact
    assert sq.item() == sq2.item()  # deterministic
    # odd offset (scalar head) gives the same sum over the same elements
    if n > 1:
        sub = gd[1:]
        exact_sub = O.grad_sqnorm(_view(gh, gk)[1:], KIND16[gk])
        assert abs(float(H.sqnorm(sub).item()) - exact_sub) <= 1e-12 * exact_sub


def test_grad_sqnorm_accumulates_over_buffers(hip_device):
    rng = np.random.default_rng(2)
    parts = [torch.from_numpy(rng.normal(0, 1e-3, k).astype(np.float32)).bfloat16() for k in (1000, 3, 77777)]
    acc = H.sqnorm(parts[0].to(hip_device))
    for t in parts[1:]:
        H.sqnorm(t.to(hip_device), accumulate_into=acc)
    exact = sum(O.grad_sqnorm(H.to_np_bits(t, "bf16"), "bf16") for t in parts)
    assert abs(acc.item() - exact) <= 1e-12 * exact


def test_clip_coef_matches_oracle_and_torch(hip_device):
    for scale, max_norm in ((1e-3, 1.0), (1e-1, 1.0), (1e-6, 1.0), (1.0, 0.5)):
        g = torch.from_numpy(np.random.default_rng(4).normal(0, scale, 300001).astype(np.float32))
        gd = g.to(hip_device)
        sq = H.sqnorm(gd)
        coef, norm = H.clip_coef(sq, max_norm)
        c_ref, n_ref = O.clip_coef(float(sq.item()), max_norm)
        assert coef.item() == np.float32(c_ref) and norm.item() == np.float32(n_ref)
        w = torch.nn.Parameter(g.clone())
        w.grad = g.clone()
        total = torch.nn.utils.clip_grad_norm_([w], max_norm)
        # torch reduces in fp32 on the GPU (relative error ~1e-6 at this length);
        # ours is the float64 sum rounded once, pinned bit-exact by the oracle above
        assert abs(total.item() - norm.item()) <= 1e-5 * norm.item()


def test_clip_non_finite_norm_propagates(hip_device):
    g = torch.zeros(1000, dtype=torch.bfloat16)
    g[10] = float("inf")
    sq = H.sqnorm(g.to(hip_device))
    coef, norm = H.clip_coef(sq, 1.0)
    assert np.isinf(norm.item()) and coef.item() == 0.0
    g[11] = float("nan")
    sq = H.sqnorm(g.to(hip_device))
    coef, norm = H.clip_coef(sq, 1.0)
    assert np.isnan(norm.item()) and np.isnan(coef.item())


def test_fused_norm_clip_reuses_workspace(hip_device):
    """la_grad_norm_clip writes sqnorm, norm and coef; back-to-back calls of
    different sizes (and so different grids) on one workspace stay exact."""
    L = H._lib.load()
    big = 16 * 1024 * 1024 + 3
    ws = torch.zeros(L.la_grad_sqnorm_workspace(big) // 8 + 1, dtype=torch.float64, device=hip_device)
    rng = np.random.default_rng(12)
    for n in (big, 5, 300_001, big, 1, 4096):
        g = torch.from_numpy(rng.normal(0, 1e-2, n).astype(np.float32)).bfloat16()
        sq, coef, norm = H.norm_clip(g.to(hip_device), 1.0, ws=ws)
        exact = O.grad_sqnorm(H.to_np_bits(g, "bf16"), "bf16")
        assert abs(sq.item() - exact) <= 1e-12 * exact
        c_ref, n_ref = O.clip_coef(sq.item(), 1.0)
        assert coef.item() == np.float32(c_ref) and norm.item() == np.float32(n_ref)


def test_norm_of_empty_buffer(hip_device):
    g = torch.zeros(0, dtype=torch.bfloat16, device=hip_device)
    sq, coef, norm = H.norm_clip(g, 1.0)
    assert sq.item() == 0.0 and norm.item() == 0.0 and coef.item() == 1.0


# ---------------------------------------------------------------------------
# configs C2 and C4 at full size
# ---------------------------------------------------------------------------

def llama8b_layer_sizes():
    h, kv, ffn = 4096, 1024, 14336
    return [h * h, h * kv, h * kv, h * h, h * ffn, h * ffn, ffn * h, h, h]


def qwen14b_layer_sizes():
    h, kv, ffn = 5120, 1024, 13824
    return [h * h, h, h * kv, kv, h * kv, kv, h * h, h * ffn, h * ffn, ffn * h, h, h]


def _dev_normal(n, std, seed, device, dtype=torch.float32):
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    return (torch.randn(n, generator=gen, device=device, dtype=torch.float32) * std).to(dtype)


def _full_size_step(n, device, *, warm_steps, wd, seed, outliers=False, max_norm=1.0, chunk=None):
    """Warm m/v with the oracle, then one clipped step on both sides; compare bits."""
    log(f"full-size n={n} warm={warm_steps} wd={wd} outliers={outliers}")
    p_d = _dev_normal(n, 0.02, seed, device)
    p_h = p_d.cpu().numpy().copy()
    m_h = np.zeros(n, np.float32)
    v_h = np.zeros(n, np.float32)
    orc = O.OracleAdam(1e-5, (0.9, 0.999), 1e-8, wd, True)
    for st in range(1, warm_steps + 1):
        g = _dev_normal(n, 1e-3, seed + st, device, torch.bfloat16)
        orc.update(st, 1e-5, 0.9, 0.999, 1e-8, wd, True, p_h, H.to_np_bits(g, "bf16"), m_h, v_h, g16="bf16")
    st = warm_steps + 1
    g = _dev_normal(n, 1e-3, seed + st, device, torch.bfloat16)
    if outliers:
        gen = torch.Generator(device=device)
        gen.manual_seed(seed + 777)
        idx = torch.randint(0, n, (n // 1000,), generator=gen, device=device)
        g[idx] = g[idx] * 100
    g_h = H.to_np_bits(g, "bf16")
    p_d = torch.from_numpy(p_h.copy()).to(device)
    m_d = torch.from_numpy(m_h.copy()).to(device)
    v_d = torch.from_numpy(v_h.copy()).to(device)
    out = torch.empty(n, dtype=torch.bfloat16, device=device)

    sq = H.sqnorm(g)
    coef, norm = H.clip_coef(sq, max_norm)
    exact = O.grad_sqnorm(g_h, "bf16")
    assert abs(sq.item() - exact) <= 1e-12 * exact
    c = float(coef.item())
    assert c < 1.0  # clipping triggers at this grad scale

    hip = H.HipAdam(1e-5, (0.9, 0.999), 1e-8, wd, True)
    # replay the warm-up calls on the host state machine (one call per step)
    for s in range(1, warm_steps + 1):
        sc = H._lib.LaScalars()
        H._lib.check(hip.L.la_scalars(hip.id, s, 1e-5, 0.9, 0.999, 1e-8, wd, 1, H.ctypes.byref(sc)), "scalars")
    chunk = chunk or n
    for lo in range(0, n, chunk):
        hi = min(lo + chunk, n)
        hip.update(st, 1e-5, 0.9, 0.999, 1e-8, wd, True, p_d[lo:hi], g[lo:hi], m_d[lo:hi], v_d[lo:hi],
                   out=out[lo:hi], coef=coef)
        orc.update(st, 1e-5, 0.9, 0.999, 1e-8, wd, True, p_h[lo:hi], g_h[lo:hi], m_h[lo:hi], v_h[lo:hi],
                   g16="bf16", clip_coef=c)
    torch.cuda.synchronize()
    assert np.array_equal(H.to_np_bits(p_d, "f32"), p_h.view(np.uint32))
    assert np.array_equal(H.to_np_bits(m_d, "f32"), m_h.view(np.uint32))
    assert np.array_equal(H.to_np_bits(v_d, "f32"), v_h.view(np.uint32))
    assert np.array_equal(H.to_np_bits(out, "bf16"), O.f32_to_bf16(p_h))


def test_c2_llama8b_layer_full_size(hip_device):
    n = sum(llama8b_layer_sizes())
    assert n == 218_112_000
    _full_size_step(n, hip_device, warm_steps=5, wd=0.01, seed=20)


@pytest.mark.parametrize("triple,mode", [(("f32", "f32", "f32"), "adamw"), (("bf16", "bf16", "bf16"), "adamw"),
                                         (("f16", "f16", "f32"), "l2"), (("bf16", "f32", "f32"), "adamw")])
def test_c2_size_other_triples(triple, mode, hip_device):
    """The reference's other registered triples (cpu_adam_impl.cpp:181-189) at the
    C2 shape (218,112,000 elements, no tail), two steps with a clip coefficient
    and the bf16 copy: every bit equals the oracle's."""
    pk, gk, sk = triple
    n = sum(llama8b_layer_sizes())
    log(f"C2-size {triple} {mode}")
    wd, adamw = (0.01, True) if mode == "adamw" else (0.01, False)
    p_d = _dev_normal(n, 0.02, 60, hip_device).to(H.TD[pk])
    m_d = torch.zeros(n, dtype=H.TD[sk], device=hip_device)
    v_d = torch.zeros(n, dtype=H.TD[sk], device=hip_device)
    out = torch.empty(n, dtype=torch.bfloat16, device=hip_device)
    p_h, m_h, v_h = H.to_np_bits(p_d, pk), H.to_np_bits(m_d, sk), H.to_np_bits(v_d, sk)
    o_h = np.zeros(n, np.uint16)
    coef = torch.tensor([0.75], device=hip_device)
    hip = H.HipAdam(1e-5, (0.9, 0.999), 1e-8, wd, adamw)
    orc = O.OracleAdam(1e-5, (0.9, 0.999), 1e-8, wd, adamw)
    for st in (1, 2):
        g = _dev_normal(n, 1e-3, 60 + st, hip_device).to(H.TD[gk])
        hip.update(st, 1e-5, 0.9, 0.999, 1e-8, wd, True, p_d, g, m_d, v_d, out=out, coef=coef)
        # the bf16 copy is RNE of the fp32 result, before any rounding to 16-bit params
        orc.update(st, 1e-5, 0.9, 0.999, 1e-8, wd, True, _view(p_h, pk), _view(H.to_np_bits(g, gk), gk),
                   _view(m_h, sk), _view(v_h, sk), p16=KIND16[pk], g16=KIND16[gk], s16=KIND16[sk],
                   clip_coef=0.75, p_bf16_out=o_h)
        del g
    torch.cuda.synchronize()
    assert np.array_equal(H.to_np_bits(p_d, pk), p_h)
    assert np.array_equal(H.to_np_bits(m_d, sk), m_h)
    assert np.array_equal(H.to_np_bits(v_d, sk), v_h)
    assert np.array_equal(H.to_np_bits(out, "bf16"), o_h)
    del p_d, m_d, v_d, out
    torch.cuda.empty_cache()


def test_c2_llama8b_layer_in_reference_chunks(hip_device):
    """The runtime's chunking: 32 Mi-element step_chunk calls (transformer_layer.py:26-27)."""
    n = sum(llama8b_layer_sizes())
    _full_size_step(n, hip_device, warm_steps=1, wd=0.01, seed=40, chunk=32 * 1024 * 1024)


def test_c4_qwen14b_layer_outliers(hip_device):
    n = sum(qwen14b_layer_sizes())
    assert n == 275_268_608
    _full_size_step(n, hip_device, warm_steps=0, wd=0.1, seed=30, outliers=True)


def test_single_call_beyond_2_pow_31_elements(hip_device):
    """64-bit indexing: one call over n = 2^31 + 2^20 + 13 elements (34 GB of HBM).
    Elements are independent given the call's scalars, so windows at the start,
    across the 2^31 boundary and at the end (holding the scalar tail) are
    checked against the oracle, each window as its own one-call step."""
    n = (1 << 31) + (1 << 20) + 13
    log(f"n={n}")
    gen = torch.Generator(device=hip_device)
    gen.manual_seed(99)
    p = torch.randn(n, generator=gen, device=hip_device) * 0.02
    g = (torch.randn(n, generator=gen, device=hip_device) * 1e-3).bfloat16()
    m = torch.zeros(n, device=hip_device)
    v = torch.zeros(n, device=hip_device)
    windows = [(0, 1 << 16), ((1 << 31) - (1 << 15), (1 << 31) + (1 << 15)), (n - (1 << 16) - 13, n)]
    before = [(p[a:b].cpu().numpy().copy(), H.to_np_bits(g[a:b], "bf16")) for a, b in windows]
    opt = H.HipAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    opt.update(1, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, p, g, m, v)
    torch.cuda.synchronize()
    for (a, b), (ph, gh) in zip(windows, before):
        assert (b - a) % 16 == (n % 16 if b == n else 0)
        mh = np.zeros(b - a, np.float32)
        vh = np.zeros(b - a, np.float32)
        orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
        orc.update(1, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, ph, gh, mh, vh, g16="bf16")
        assert np.array_equal(H.to_np_bits(p[a:b], "f32"), ph.view(np.uint32)), (a, b)
        assert np.array_equal(H.to_np_bits(m[a:b], "f32"), mh.view(np.uint32)), (a, b)
        assert np.array_equal(H.to_np_bits(v[a:b], "f32"), vh.view(np.uint32)), (a, b)
    del p, g, m, v
    torch.cuda.empty_cache()


# ---------------------------------------------------------------------------
# several calls of one step in one launch (la_adam_update_multi)
# ---------------------------------------------------------------------------

# the last size: a 4 Mi-element segment batched with the small ones
MULTI_SIZES = [1, 3, 15, 16, 17, 255, 256, 257, 4099, 100_003, 7, 64, 1000, 33, 2, 5000, 12, 129, 31, 8,
               16384 * 256 + 101]


@pytest.mark.parametrize("mode", ["adamw", "l2", "none"])
@pytest.mark.parametrize("triple", [("f32", "bf16", "f32"), ("f32", "f32", "f32"), ("bf16", "bf16", "bf16")])
def test_multi_update_equals_separate_calls(triple, mode, hip_device):
    """21 segments of awkward sizes: 19 small ones and a 4 Mi-element one (two
    batched launches of up to 16) and one whose params are out of phase with
    its grads (launched on its own).  Some sit at odd
    element offsets inside their buffers; a clip coefficient applies and every
    other segment writes a bf16 copy.  Bit-exact with the same 21
    la_adam_update calls, and every segment with the oracle replaying them."""
    pk, gk, sk = triple
    td = {"f32": torch.float32, "bf16": torch.bfloat16}
    log(f"multi-update {triple} {mode}")
    wd = 0.0 if mode == "none" else 0.01
    adamw = mode != "l2"
    coef = torch.tensor([0.37], device=hip_device)

    def make():
        torch.manual_seed(11)
        segs = []
        for k, n in enumerate(MULTI_SIZES):
            off = (k * 3) % 4                                 # odd offsets inside a larger buffer
            goff = (off + 1) % 4 if k == 9 else off           # segment 9: params out of phase with grads
            def buf(dt, o, std):
                return (torch.randn(n + 8, device=hip_device) * std).to(td[dt])[o:o + n]
            p = buf(pk, off, 0.02)
            g = buf(gk, goff, 1e-3)
            m = buf(sk, off, 1e-3)
            v = buf(sk, off, 1e-3).abs_()
            out = torch.empty(n + 4, dtype=torch.bfloat16, device=hip_device)[off:off + n] if k % 2 else None
            segs.append([p, g, m, v, out])
        return segs

    a, b = make(), make()
    opt_a = H.HipAdam(1e-3, (0.9, 0.999), 1e-8, wd, adamw)
    opt_b = H.HipAdam(1e-3, (0.9, 0.999), 1e-8, wd, adamw)
    for step in (1, 2, 3):
        opt_a.update_multi(step, 1e-3, 0.9, 0.999, 1e-8, wd, True, a, coef=coef)
        for p, g, m, v, out in b:
            opt_b.update(step, 1e-3, 0.9, 0.999, 1e-8, wd, True, p, g, m, v, out=out, coef=coef)
    torch.cuda.synchronize()
    for k, (sa, sb) in enumerate(zip(a, b)):
        for i, kind in enumerate((pk, sk, sk)):
            assert np.array_equal(H.to_np_bits(sa[(0, 2, 3)[i]], kind), H.to_np_bits(sb[(0, 2, 3)[i]], kind)), (k, i)
        if sa[4] is not None:
            assert np.array_equal(H.to_np_bits(sa[4], "bf16"), H.to_np_bits(sb[4], "bf16")), k
    # absolute check against the oracle, replaying the same 21 calls per step
    c = make()
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, wd, adamw)
    hp = [H.to_np_bits(s[0], pk) for s in c]
    hm = [H.to_np_bits(s[2], sk) for s in c]
    hv = [H.to_np_bits(s[3], sk) for s in c]
    hg = [H.to_np_bits(s[1], gk) for s in c]
    for step in (1, 2, 3):
        for k in range(len(c)):
            orc.update(step, 1e-3, 0.9, 0.999, 1e-8, wd, True, _view(hp[k], pk), _view(hg[k], gk),
                       _view(hm[k], sk), _view(hv[k], sk), p16=KIND16[pk], g16=KIND16[gk], s16=KIND16[sk],
                       clip_coef=0.37)
    for k in range(len(c)):
        assert np.array_equal(H.to_np_bits(a[k][0], pk), hp[k]), k
        assert np.array_equal(H.to_np_bits(a[k][2], sk), hm[k]), k
        assert np.array_equal(H.to_np_bits(a[k][3], sk), hv[k]), k


# ---------------------------------------------------------------------------
# launch paths the product build takes only at sizes beyond one GPU: the
# small-grid test build (64 waves per update launch, 2 workgroups per norm
# launch, so at most 32 runs per multi batch and an own grid-stride launch for
# a segment of more runs, which the product build gives a segment whose
# pointers agree in phase only above 2^33 elements) against the product build
# ---------------------------------------------------------------------------

SMALL_GRID_SIZES = [7, 16, 64 * 256 * 3 + 5, 64 * 256 * 40 + 13, 1_000_003]


@pytest.mark.parametrize("triple", [("f32", "bf16", "f32"), ("bf16", "bf16", "bf16"), ("f16", "f16", "f32")])
def test_grid_stride_update_equals_one_shot(triple, hip_device):
    """The update kernel's grid-stride loop (several trips of 64 waves) and its
    scalar head/tail loop, in the small-grid build, give the same bits as the
    product build's one-shot grid, with a bf16 copy and a clip coefficient,
    over three steps; the multi-segment entry point likewise, where every
    segment of more than 32 runs (8192 elements: more than one batch of the
    small-grid build holds) takes its own grid-stride launch and the small
    ones share batches.  The
    product build is itself pinned to the oracle by the tests above; the
    small-grid results are also checked against the oracle here."""
    pk, gk, sk = triple
    log(f"grid-stride update {triple}")
    small = H.load_small_grid()
    coef = torch.tensor([0.61], device=hip_device)

    def make(seed):
        torch.manual_seed(seed)
        out = []
        for n in SMALL_GRID_SIZES:
            off = n % 3                                        # element offsets inside a larger buffer
            def buf(dt, std):
                return (torch.randn(n + 4, device=hip_device) * std).to(H.TD[dt])[off:off + n]
            # every stream at the same element offset: the vector path, not the all-scalar one
            out.append([buf(pk, 0.02), buf(gk, 1e-3), buf(sk, 1e-3), buf(sk, 1e-3).abs_(),
                        torch.empty(n + 4, dtype=torch.bfloat16, device=hip_device)[off:off + n]])
        return out

    for multi in (False, True):
        a, b = make(5), make(5)
        opt_a = H.HipAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True, lib=small)
        opt_b = H.HipAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
        for step in (1, 2, 3):
            if multi:
                opt_a.update_multi(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, a, coef=coef)
                opt_b.update_multi(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, b, coef=coef)
            else:
                for (p, g, m, v, o), (q, h, mm, vv, oo) in zip(a, b):
                    opt_a.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, p, g, m, v, out=o, coef=coef)
                    opt_b.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, q, h, mm, vv, out=oo, coef=coef)
        torch.cuda.synchronize()
        for k, (sa, sb) in enumerate(zip(a, b)):
            for i, kind in ((0, pk), (2, sk), (3, sk), (4, "bf16")):
                assert np.array_equal(H.to_np_bits(sa[i], kind), H.to_np_bits(sb[i], kind)), (multi, k, i)
    # against the oracle, replaying the same five calls per step in order: the
    # beta-power state takes the multiply path on a step's first call and the
    # pow path on the others (cpu_adam.h:57-89), which changes step_size bits
    host = [[H.to_np_bits(t, kind) for t, kind in zip(seg[:4], (pk, gk, sk, sk))] for seg in make(5)]
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    for step in (1, 2, 3):
        for p, g, m, v in host:
            orc.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, _view(p, pk), _view(g, gk), _view(m, sk),
                       _view(v, sk), p16=KIND16[pk], g16=KIND16[gk], s16=KIND16[sk], clip_coef=0.61)
    for k, (p, g, m, v) in enumerate(host):
        assert np.array_equal(H.to_np_bits(a[k][0], pk), p), k
        assert np.array_equal(H.to_np_bits(a[k][2], sk), m), k
        assert np.array_equal(H.to_np_bits(a[k][3], sk), v), k


@pytest.mark.parametrize("gk", ["bf16", "f32", "f16"])
def test_grad_norm_with_two_workgroups(gk, hip_device):
    """The grad norm's stage 1 with a two-workgroup grid (many trips of the
    unrolled loop, then its remainder and the head/tail elements) stays within
    1e-12 of the oracle's compensated float64 sum, at sizes around one trip."""
    import ctypes

    small = H.load_small_grid()
    log(f"two-workgroup norm {gk}")
    trip = 2 * 512 * 8 * 4                                     # elements per trip of the unrolled loop
    for n in (1, 3, trip - 1, trip, trip + 5, 7 * trip + 1001, 1_000_003):
        g = (torch.randn(n + 2, device=hip_device) * 1e-2).to(H.TD[gk])[1:1 + n]
        ws = torch.zeros(small.la_grad_sqnorm_workspace(n) // 8 + 1, dtype=torch.float64, device=hip_device)
        assert small.la_grad_sqnorm_workspace(n) <= 2 * 8
        out = torch.zeros(1, dtype=torch.float64, device=hip_device)
        rc = small.la_grad_sqnorm(H.CODE[gk], ctypes.c_void_p(g.data_ptr()), n, ctypes.c_void_p(ws.data_ptr()),
                                  ws.numel() * 8, ctypes.c_void_p(out.data_ptr()), 0,
                                  torch.cuda.current_stream(hip_device).cuda_stream)
        assert rc == 0
        exact = O.grad_sqnorm(_view(H.to_np_bits(g, gk), gk), KIND16[gk])
        assert abs(out.item() - exact) <= 1e-12 * exact, (n, out.item(), exact)


# ---------------------------------------------------------------------------
# the C-ABI from a plain C program (no torch, no Python in the process)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("alloc", ["hipMalloc", "vmm"])
def test_plain_c_program_runs_the_step(alloc, tmp_path):
    """tests/native/device_from_c.c (built by slideformer_amd.build) computes the
    clip coefficient and three clipped AdamW steps with the bf16 copy through
    include/layer_adam.h and the HIP runtime API alone; every output bit
    equals the oracle's.  Its device arrays come from hipMalloc, or from HIP
    virtual memory (hipMemAddressReserve / hipMemCreate / hipMemMap), the kind
    of mapping an allocator with expandable segments hands out; torch's ROCm
    build does not offer expandable segments on this platform, so the program
    maps the memory itself."""
    import os
    import subprocess

    from slideformer_amd.build import C_DRIVER
    assert os.path.exists(C_DRIVER), "run `python -m slideformer_amd.build` first"
    n = 100_003
    rng = np.random.default_rng(404)
    p = rng.normal(0, 0.02, n).astype(np.float32)
    g = O.f32_to_bf16(rng.normal(0, 1e-2, n).astype(np.float32))
    m = rng.normal(0, 1e-3, n).astype(np.float32)
    v = np.abs(rng.normal(0, 1e-6, n)).astype(np.float32)
    src, dst = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(src, "wb") as f:
        f.write(np.uint64(n).tobytes() + p.tobytes() + g.tobytes() + m.tobytes() + v.tobytes())
    log(f"device_from_c n={n} {alloc}")
    res = subprocess.run([C_DRIVER, str(src), str(dst)] + (["vmm"] if alloc == "vmm" else []), capture_output=True,
                         text=True, timeout=120)
    if res.returncode == 30:
        pytest.skip("the device does not support HIP virtual memory")
    assert res.returncode == 0, (res.returncode, res.stderr)
    assert alloc != "vmm" or "virtual-memory arrays" in res.stdout
    raw = np.fromfile(dst, dtype=np.uint8)
    coef, norm = np.frombuffer(raw[:8].tobytes(), dtype=np.float32)
    body = raw[8:]
    gp = np.frombuffer(body[:4 * n].tobytes(), dtype=np.float32)
    gm = np.frombuffer(body[4 * n:8 * n].tobytes(), dtype=np.float32)
    gv = np.frombuffer(body[8 * n:12 * n].tobytes(), dtype=np.float32)
    gout = np.frombuffer(body[12 * n:14 * n].tobytes(), dtype=np.uint16)
    c_ref, n_ref = O.clip_coef(O.grad_sqnorm(g, "bf16"), 0.5)
    assert coef == np.float32(c_ref) and norm == np.float32(n_ref) and coef < 1.0
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    for step in (1, 2, 3):
        orc.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, p, g, m, v, g16="bf16", clip_coef=float(coef))
    assert np.array_equal(gp.view(np.uint32), p.view(np.uint32))
    assert np.array_equal(gm.view(np.uint32), m.view(np.uint32))
    assert np.array_equal(gv.view(np.uint32), v.view(np.uint32))
    assert np.array_equal(gout, O.f32_to_bf16(p))


def test_bf16_copy_rounding_of_every_fp32_bit_pattern(hip_device):
    """The bf16 compute copy, brute force over all 2^32 fp32 bit patterns: with
    lr = 0, zero grads and zero moments the update leaves every master value
    as it is (p + 0 * -0), so the copy the kernel writes is the rounding of an
    arbitrary fp32 input.  It must equal the reference's bf16 store,
    (u + 0x7FFF + ((u >> 16) & 1)) >> 16 with NaN -> 0x7FC0 (simd.h:56-86),
    for every input; computed on the device in 16 launches of 2^28."""
    chunk = 1 << 28
    hip = H.HipAdam(0.0, (0.9, 0.999), 1e-8, 0.0, True)
    g = torch.zeros(chunk, dtype=torch.bfloat16, device=hip_device)
    m = torch.zeros(chunk, device=hip_device)
    v = torch.zeros(chunk, device=hip_device)
    out = torch.empty(chunk, dtype=torch.bfloat16, device=hip_device)
    for c in range(16):
        log(f"bf16 rounding, patterns [{c * chunk:#x}, {(c + 1) * chunk:#x})")
        bits = torch.arange(c * chunk, (c + 1) * chunk, dtype=torch.int64, device=hip_device)
        p = bits.to(torch.int32).view(torch.float32)       # wraps to the int32 bit pattern
        del bits
        m.zero_()
        v.zero_()
        hip.update(c + 1, 0.0, 0.9, 0.999, 1e-8, 0.0, True, p, g, m, v, out=out)
        u = p.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
        want = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
        want = torch.where((u & 0x7FFFFFFF) > 0x7F800000, torch.full_like(want, 0x7FC0), want)
        got = out.view(torch.int16).to(torch.int64) & 0xFFFF
        bad = int((got != want).sum().item())
        assert bad == 0, (c, bad)
        # the master itself is unchanged (NaN stays NaN)
        orig = torch.arange(c * chunk, (c + 1) * chunk, dtype=torch.int64, device=hip_device)
        same = (u == (orig & 0xFFFFFFFF)) | ((u & 0x7FFFFFFF) > 0x7F800000)
        assert bool(same.all()), c
        del p, u, want, got, orig, same
    torch.cuda.empty_cache()


def test_fp16_store_rounding_of_every_fp32_bit_pattern(hip_device):
    """The fp16 store (hardware conversion behind an opaque value), brute force
    over all 2^32 fp32 bit patterns via the (f16, f32, f32) triple: with lr 1,
    betas (0, 1), eps 0, no decay and no bias correction, p = 0, m = 0, v = 1,
    the update computes m = g, v = 1, d = 1, u = g and p = fma(u, -1, 0) = -g
    exactly, then stores p as fp16.  That must equal the CPU's IEEE
    round-to-nearest-even of the same fp32 value (0 + -g; torch's CPU
    conversion, the x86 F16C instruction), NaN as a class.
    Patterns with |g| >= 2^63 are left out: there g*g overflows and v turns
    NaN (every fp16 of them would be +-inf anyway)."""
    chunk = 1 << 28
    hip = H.HipAdam(1.0, (0.0, 1.0), 0.0, 0.0, True)
    p = torch.zeros(chunk, dtype=torch.float16, device=hip_device)
    m = torch.zeros(chunk, device=hip_device)
    v = torch.ones(chunk, device=hip_device)
    checked = 0
    for c in range(16):
        log(f"fp16 rounding, patterns [{c * chunk:#x}, {(c + 1) * chunk:#x})")
        g = torch.arange(c * chunk, (c + 1) * chunk, dtype=torch.int64, device=hip_device).to(
            torch.int32).view(torch.float32)
        p.zero_()
        m.zero_()
        v.fill_(1.0)
        hip.update(c + 1, 1.0, 0.0, 1.0, 0.0, 0.0, False, p, g, m, v)
        g_h = g.cpu()
        got = p.cpu()
        want = (torch.zeros((), dtype=torch.float32) + (-g_h)).to(torch.float16)
        skip = g_h.abs() >= 2.0 ** 63                       # NaN compares false: kept
        nan = want.isnan()
        assert bool(((got.isnan() == nan) | skip).all()), c
        assert bool(((got.view(torch.int16) == want.view(torch.int16)) | skip | nan).all()), c
        checked += g_h.numel() - int(skip.sum())
        del g, g_h, got, want, skip, nan
    assert checked > (1 << 32) - (1 << 31)
    torch.cuda.empty_cache()


def test_bf16_master_store_rounding_of_every_fp32_bit_pattern(hip_device):
    """The bf16 store of the master itself (not the copy stream), brute force
    over all 2^32 fp32 bit patterns via the (bf16, f32, f32) triple, set up as
    in the fp16 test above: the update computes p = fma(g, -1, +0), which is
    -g exactly except that both zeros give +0, then stores p as bf16.  That
    must equal the reference's bf16 store (simd.h:56-86) of the same value,
    (u + 0x7FFF + ((u >> 16) & 1)) >> 16 with NaN -> 0x7FC0, for every input,
    NaN grads included (they make p NaN).  Finite patterns with |g| >= 2^63
    are left out: there g*g overflows, v turns NaN and so does p.  The
    expected bits are integer arithmetic on the device."""
    chunk = 1 << 28
    hip = H.HipAdam(1.0, (0.0, 1.0), 0.0, 0.0, True)
    p = torch.zeros(chunk, dtype=torch.bfloat16, device=hip_device)
    m = torch.zeros(chunk, device=hip_device)
    v = torch.ones(chunk, device=hip_device)
    checked = 0
    for c in range(16):
        log(f"bf16 master rounding, patterns [{c * chunk:#x}, {(c + 1) * chunk:#x})")
        u = torch.arange(c * chunk, (c + 1) * chunk, dtype=torch.int64, device=hip_device)
        g = u.to(torch.int32).view(torch.float32)
        p.zero_()
        m.zero_()
        v.fill_(1.0)
        hip.update(c + 1, 1.0, 0.0, 1.0, 0.0, 0.0, False, p, g, m, v)
        mag = u & 0x7FFFFFFF
        x = torch.where(mag == 0, torch.zeros_like(u), u ^ 0x80000000)          # 0 + -g
        want = ((x + 0x7FFF + ((x >> 16) & 1)) >> 16) & 0xFFFF
        want = torch.where(mag > 0x7F800000, torch.full_like(want, 0x7FC0), want)
        keep = (mag < 0x5F000000) | (mag > 0x7F800000)                             # |g| < 2^63, or NaN
        got = p.view(torch.int16).to(torch.int64) & 0xFFFF
        bad = int(((got != want) & keep).sum().item())
        assert bad == 0, (c, bad)
        checked += int(keep.sum().item())
        del u, g, mag, x, want, keep, got
    assert checked > (1 << 32) - (1 << 31)
    torch.cuda.empty_cache()


def test_sqrt_and_divide_over_fp32_bit_patterns(hip_device):
    """The kernel's correctly rounded sqrt and division over fp32 bit patterns
    of v via the (f32, f32, f32) triple: with lr 1, betas (0, 1), eps 0, no
    decay, no bias correction, g = 1, m = 0, p = 0 the body computes m = 1,
    v' = v * 1 + 1 * 0, d = sqrt(v') * 1 + 0, u = m / d and p = u * -1 + 0
    (cpu_adam.h:159-192).  Patterns, both signs: every one with exponent field
    0 or 1 (denormals and the smallest normals), every one with exponent field
    0xFE or 0xFF (the largest normals, Inf, NaN), and every 61st of the rest.
    The CPU computes the same sequence in float64 and rounds to float32 once
    per operation; float64 carries 53 >= 2 x 24 + 2 bits, so that equals the
    correctly rounded float32 sqrt and division.  (torch's own CPU float32
    sqrt is not correctly rounded: it differs from numpy's float32 sqrt on
    about 0.6 % of random inputs, so it cannot serve here.)  Every bit of p
    must match, NaN as a class."""
    parts = []
    for sign in (0, 1 << 31):
        parts.append(torch.arange(0, 1 << 24, dtype=torch.int64) + sign)                 # exponent 0, 1
        parts.append(torch.arange(0xFE << 23, 1 << 31, dtype=torch.int64) + sign)         # exponent 0xFE, 0xFF
    parts.append(torch.arange(1 << 24, 1 << 32, 61, dtype=torch.int64))                  # the rest, both signs
    pats = torch.cat(parts)
    n = pats.numel()
    log(f"sqrt/divide over {n} patterns")
    v_h = pats.to(torch.int32).view(torch.float32)
    del parts, pats
    hip = H.HipAdam(1.0, (0.0, 1.0), 0.0, 0.0, True)
    v = v_h.to(hip_device)
    p = torch.zeros(n, device=hip_device)
    m = torch.zeros(n, device=hip_device)
    g = torch.ones(n, device=hip_device)
    hip.update(1, 1.0, 0.0, 1.0, 0.0, 0.0, False, p, g, m, v)
    got = p.cpu()
    log("GPU done; CPU reference")
    v1 = (v_h.to(torch.float64) * 1.0 + 0.0).to(torch.float32)
    d = (torch.sqrt(v1.to(torch.float64)).to(torch.float32).to(torch.float64) * 1.0 + 0.0).to(torch.float32)
    u = (1.0 / d.to(torch.float64)).to(torch.float32)
    want = (0.0 + -u.to(torch.float64)).to(torch.float32)
    nan = want.isnan()
    assert bool((got.isnan() == nan).all())
    assert bool(((got.view(torch.int32) == want.view(torch.int32)) | nan).all())
    del v, p, m, g, got, v_h, v1, d, u, want, nan
    torch.cuda.empty_cache()


@pytest.mark.parametrize("pk,gk", [("f16", "f16"), ("bf16", "bf16")])
def test_16bit_params_of_every_pattern_round_trip(pk, gk, hip_device):
    """Every one of the 65,536 fp16 / bf16 patterns as a 16-bit master, with
    lr 0, zero grads and zero fp32 moments (the (f16, f16, f32) and
    (bf16, bf16, f32) triples): the update leaves the value as it is, so the
    stored master equals its input bit for bit (NaN as a class), and the bf16
    copy is the bf16 rounding of the exactly widened input (numpy's float16
    widening, the reference's bf16 formula in the oracle)."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    p = H.to_dev_bits(bits, pk, hip_device)
    g = torch.zeros(bits.size, dtype=H.TD[gk], device=hip_device)
    m = torch.zeros(bits.size, device=hip_device)
    v = torch.zeros(bits.size, device=hip_device)
    out = torch.empty(bits.size, dtype=torch.bfloat16, device=hip_device)
    hip = H.HipAdam(0.0, (0.9, 0.999), 1e-8, 0.0, True)
    hip.update(1, 0.0, 0.9, 0.999, 1e-8, 0.0, True, p, g, m, v, out=out)
    torch.cuda.synchronize()
    got = H.to_np_bits(p, pk)
    wide = bits.view(np.float16).astype(np.float32) if pk == "f16" else O.bf16_to_f32(bits)
    nan = np.isnan(wide)
    assert np.array_equal(got[~nan], bits[~nan])
    got_f = got.view(np.float16).astype(np.float32) if pk == "f16" else O.bf16_to_f32(got)
    assert np.isnan(got_f[nan]).all()
    o = H.to_np_bits(out, "bf16")
    want = O.f32_to_bf16(wide)
    assert np.array_equal(o[~nan], want[~nan])
    assert (o[nan] == 0x7FC0).all()
