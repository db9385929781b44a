"""Pins the CPU checker (oracle/) before anything is compared against it.

- every golden case written by the reference compiled from its own sources
  (tests/golden/make_golden.py) is reproduced bit for bit;
- where oracle/_ref is built here, direct bit-exact comparisons on fresh inputs;
- the known-answer test of the reference (test_shared_data_parallel.py:53-93)
  against torch.optim.AdamW;
- conversions against torch / numpy, the norm against exact float64 sums,
  the clip coefficient against torch.nn.utils.clip_grad_norm_;
- planted mistakes in the oracle fail the fixtures.
"""
from __future__ import annotations

import math
import zlib

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests import _golden as G

KIND16 = {"bf16": "bf16", "f16": "f16", "f32": None}


def _view(bits_arr, kind):
    return bits_arr.view(np.float32) if kind == "f32" else bits_arr


def oracle_updater(meta, body_width=16):
    pk, gk, sk = meta["triple"]
    b1, b2 = meta["betas"]
    opt = O.OracleAdam(1e-3, (b1, b2), meta["eps"], meta["wd"], meta["adamw"])

    def call(step, lr, p, g, m, v, lo, hi):
        opt.update(step, lr, b1, b2, meta["eps"], meta["wd"], meta["bc"],
                   _view(p, pk)[lo:hi], _view(g, gk)[lo:hi], _view(m, sk)[lo:hi], _view(v, sk)[lo:hi],
                   p16=KIND16[pk], g16=KIND16[gk], s16=KIND16[sk], body_width=body_width)
    return call


@pytest.mark.parametrize("name", G.case_names())
def test_oracle_reproduces_golden(name):
    meta, arrays = G.get_case(name)
    got = G.replay(meta, arrays, oracle_updater(meta))
    assert G.mismatches(meta, arrays, got) == (0, 0, 0)


def test_planted_tail_order_mistake_is_caught():
    # the body op order applied to the scalar tail must disagree with the fixtures
    meta, arrays = G.get_case("tail_hot")
    got = G.replay(meta, arrays, oracle_updater(meta, body_width=1))
    assert sum(G.mismatches(meta, arrays, got)) > 0


def test_planted_all_scalar_mistake_is_caught():
    meta, arrays = G.get_case("tail_f32")
    got = G.replay(meta, arrays, oracle_updater(meta, body_width=0))
    assert sum(G.mismatches(meta, arrays, got)) > 0


def test_state_machine_paths_differ():
    """The multiply path and the pow path give different beta powers somewhere,
    so the bc_* fixtures discriminate between them."""
    a = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.0, True)
    b = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.0, True)
    lib = O.lib()
    diffs = 0
    for st in range(1, 300):
        lib.orc_increment_step(a.s, st, 0.9, 0.999)           # multiply path
        lib.orc_increment_step(b.s, st, 0.9, 0.999)
        lib.orc_increment_step(b.s, st, 0.9, 0.999)           # second call: pow path
        diffs += (a.s.betta2_t != b.s.betta2_t) or (a.s.betta1_t != b.s.betta1_t)
    assert diffs > 0


# ---------------------------------------------------------------------------
# direct comparison with the compiled reference (only where it is built)
# ---------------------------------------------------------------------------

def _ref_or_skip():
    ref = O.load_ref()
    if ref is None:
        pytest.skip("oracle/_ref not built on this host")
    return ref


TRIPLES = [("f32", "bf16", "f32"), ("f32", "f32", "f32"), ("f32", "f16", "f32"),
           ("bf16", "bf16", "f32"), ("bf16", "f32", "f32"), ("bf16", "bf16", "bf16"),
           ("f16", "f16", "f32"), ("f16", "f32", "f32"), ("f16", "f16", "f16")]
TD = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _np_bits(t, kind):
    if kind == "f32":
        return t.view(torch.int32).numpy().view(np.uint32).copy()
    return t.view(torch.int16).numpy().view(np.uint16).copy()


@pytest.mark.parametrize("triple", TRIPLES)
@pytest.mark.parametrize("mode", ["adamw", "l2", "none"])
def test_oracle_matches_compiled_reference(triple, mode):
    ref = _ref_or_skip()
    pk, gk, sk = triple
    wd = 0.0 if mode == "none" else 0.05
    adamw = mode != "l2"
    rng = np.random.default_rng(zlib.crc32(repr((triple, mode)).encode()))
    sizes = (100003, 16, 7)
    n = sum(sizes)
    p = torch.from_numpy(rng.normal(0, 0.02, n).astype(np.float32)).to(TD[pk])
    m = torch.zeros(n, dtype=TD[sk])
    v = torch.zeros(n, dtype=TD[sk])
    pb, mb, vb = _np_bits(p, pk), _np_bits(m, sk), _np_bits(v, sk)
    ref.create_adam(0, 1e-3, 0.9, 0.999, 1e-8, wd, adamw, False)
    opt = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, wd, adamw)
    for st in range(1, 4):
        g = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).to(TD[gk])
        gb = _np_bits(g, gk)
        lo = 0
        for size in sizes:
            hi = lo + size
            ref.adam_update(0, st, 1e-3, 0.9, 0.999, 1e-8, wd, True, p[lo:hi], g[lo:hi], m[lo:hi], v[lo:hi])
            opt.update(st, 1e-3, 0.9, 0.999, 1e-8, wd, True, _view(pb, pk)[lo:hi], _view(gb, gk)[lo:hi],
                       _view(mb, sk)[lo:hi], _view(vb, sk)[lo:hi], p16=KIND16[pk], g16=KIND16[gk],
                       s16=KIND16[sk])
            lo = hi
    assert G.same_bits(_np_bits(p, pk), pb, pk).all()
    assert G.same_bits(_np_bits(m, sk), mb, sk).all()
    assert G.same_bits(_np_bits(v, sk), vb, sk).all()


AVX2_WIDTH = [(("f32", "bf16", "f32"), 0), (("bf16", "bf16", "bf16"), 0), (("f32", "f32", "f32"), 8),
              (("f16", "f16", "f16"), 8), (("f32", "f16", "f32"), 8)]


@pytest.mark.parametrize("triple,width", AVX2_WIDTH, ids=lambda x: "-".join(x) if isinstance(x, tuple) else str(x))
def test_oracle_body_width_matches_the_avx2_reference_build(triple, width):
    """The reference's SIMD width follows the host ISA (builder.py:55-82,
    simd.h:32-45,95-108): 16 lanes with AVX-512, 8 with AVX2 only.  Without
    AVX-512, Step_AVX returns before its body for any triple with a bf16
    operand (cpu_adam.h:117-122), so rounded_size stays 0 and every element
    takes the scalar loop (cpu_adam_impl.cpp:29-34): the oracle's body_width=0.
    The f32/f16 triples run the 8-lane body with an n mod 8 scalar tail.  The
    AVX2 build compiled from the same sources (oracle/Makefile) must equal the
    oracle at that width and differ from it at the others, on call sizes with
    every tail length 0-15 and non-zero moments.  The product follows the
    AVX-512 build (body_width=16)."""
    if "avx2" not in O._cpu_flags() or "fma" not in O._cpu_flags():
        pytest.skip("host cannot run the AVX2 build")
    ref = O.load_ref("avx2")
    if ref is None:
        pytest.skip("oracle/_ref AVX2 build not present")
    pk, gk, sk = triple
    rng = np.random.default_rng(zlib.crc32(repr(triple).encode()))
    sizes = tuple(64 + t for t in range(16)) + (4099,)
    n = sum(sizes)
    p0 = torch.from_numpy(rng.normal(0, 0.02, n).astype(np.float32)).to(TD[pk])
    m0 = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).to(TD[sk])
    v0 = torch.from_numpy(np.abs(rng.normal(0, 1e-3, n)).astype(np.float32) ** 2).to(TD[sk])
    grads = [torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).to(TD[gk]) for _ in range(2)]

    p, m, v = p0.clone(), m0.clone(), v0.clone()
    ref.create_adam(0, 1e-3, 0.9, 0.999, 1e-8, 0.05, True, False)
    for st, g in enumerate(grads, start=1):
        lo = 0
        for size in sizes:
            hi = lo + size
            ref.adam_update(0, st, 1e-3, 0.9, 0.999, 1e-8, 0.05, True, p[lo:hi], g[lo:hi], m[lo:hi], v[lo:hi])
            lo = hi
    expect = (_np_bits(p, pk), _np_bits(m, sk), _np_bits(v, sk))

    def oracle_at(bw):
        pb, mb, vb = _np_bits(p0, pk), _np_bits(m0, sk), _np_bits(v0, sk)
        opt = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.05, True)
        for st, g in enumerate(grads, start=1):
            gb = _np_bits(g, gk)
            lo = 0
            for size in sizes:
                hi = lo + size
                opt.update(st, 1e-3, 0.9, 0.999, 1e-8, 0.05, True, _view(pb, pk)[lo:hi], _view(gb, gk)[lo:hi],
                           _view(mb, sk)[lo:hi], _view(vb, sk)[lo:hi], p16=KIND16[pk], g16=KIND16[gk],
                           s16=KIND16[sk], body_width=bw)
                lo = hi
        return pb, mb, vb

    def same(got):
        return all(G.same_bits(e, o, k).all() for e, o, k in zip(expect, got, (pk, sk, sk)))

    assert same(oracle_at(width))
    # the inputs tell the widths apart: the scalar-only and 16-lane semantics
    # give other bits than the 8-lane build and vice versa
    others = [bw for bw in (0, 8, 16) if bw != width]
    assert not same(oracle_at(others[0]))
    if sk == "f32":
        assert not same(oracle_at(others[1]))


def test_oracle_clip_equals_reference_on_prescaled_grads():
    """clip_coef inside the oracle == the reference fed fl32(f32(g)*coef) through
    its (float, float, float) triple (cpu_adam_impl.cpp:187)."""
    ref = _ref_or_skip()
    rng = np.random.default_rng(7)
    n = 4099
    coef = np.float32(0.0679)
    p = torch.from_numpy(rng.normal(0, 0.02, n).astype(np.float32))
    m, v = torch.zeros(n), torch.zeros(n)
    pb, mb, vb = p.numpy().copy(), m.numpy().copy(), v.numpy().copy()
    ref.create_adam(0, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, False)
    opt = O.OracleAdam(1e-5, (0.9, 0.999), 1e-8, 0.01, True)
    for st in range(1, 4):
        g = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).bfloat16()
        g_scaled = g.float() * float(coef)
        ref.adam_update(0, st, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, p, g_scaled, m, v)
        opt.update(st, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, pb, _np_bits(g, "bf16"), mb, vb,
                   g16="bf16", clip_coef=float(coef))
    assert np.array_equal(p.numpy().view(np.uint32), pb.view(np.uint32))
    assert np.array_equal(m.numpy().view(np.uint32), mb.view(np.uint32))
    assert np.array_equal(v.numpy().view(np.uint32), vb.view(np.uint32))


# ---------------------------------------------------------------------------
# known-answer test of the reference, test_shared_data_parallel.py:53-93
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("gdtype", [torch.float32, torch.bfloat16])
def test_oracle_known_answer_vs_torch_adamw(gdtype):
    sizes, chunk = (19, 3, 0), 5
    opt = O.OracleAdam(0.01, (0.8, 0.95), 1e-6, 0.1, True)
    for layer, size in enumerate(sizes):
        initial = torch.linspace(-0.5, 0.5, size)
        params = initial.clone().numpy()
        m = np.zeros(size, np.float32)
        v = np.zeros(size, np.float32)
        reference = torch.nn.Parameter(initial.clone())
        tadam = torch.optim.AdamW([reference], lr=0.01, betas=(0.8, 0.95), eps=1e-6,
                                  weight_decay=0.1, foreach=False)
        for step in range(1, 6):
            grad = ((torch.arange(size) * 0.13 + step * 0.2).sin() * 0.1).to(gdtype)
            lr = 0.01 if step < 3 else 0.003
            tadam.param_groups[0]["lr"] = lr
            gb = grad.float().numpy().copy() if gdtype == torch.float32 else _np_bits(grad, "bf16")
            for start in range(0, size, chunk):
                end = min(start + chunk, size)
                opt.update(step, lr, 0.8, 0.95, 1e-6, 0.1, True, params[start:end], gb[start:end],
                           m[start:end], v[start:end], g16="bf16" if gdtype == torch.bfloat16 else None)
            reference.grad = grad.float()
            tadam.step()
            torch.testing.assert_close(torch.from_numpy(params), reference.detach(), rtol=1e-6, atol=1e-7)
            st = tadam.state[reference]
            torch.testing.assert_close(torch.from_numpy(m), st["exp_avg"])
            torch.testing.assert_close(torch.from_numpy(v), st["exp_avg_sq"])


def test_oracle_tiny_vs_float64_closed_form():
    """Brute force in float64 on tiny inputs (sanity of every term)."""
    rng = np.random.default_rng(3)
    n, lr, b1, b2, eps, wd = 37, 1e-3, 0.9, 0.999, 1e-8, 0.01
    # the reference receives the hyper-parameters as C floats (cpu_adam.h:199-221)
    f = lambda x: float(np.float32(x))  # noqa: E731
    lr64, b164, b264, eps64, wd64 = f(lr), f(b1), f(b2), f(eps), f(wd)
    p = rng.normal(0, 0.02, n).astype(np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    p64, m64, v64 = p.astype(np.float64), m.astype(np.float64), v.astype(np.float64)
    opt = O.OracleAdam(lr, (b1, b2), eps, wd, True)
    for st in range(1, 6):
        g = rng.normal(0, 1e-3, n).astype(np.float32)
        opt.update(st, lr, b1, b2, eps, wd, True, p, g.copy(), m, v)
        g64 = g.astype(np.float64)
        m64 = b164 * m64 + (1 - b164) * g64
        v64 = b264 * v64 + (1 - b264) * g64 * g64
        p64 = p64 * (1 - lr64 * wd64)
        p64 = p64 - lr64 / (1 - b164 ** st) * m64 / (np.sqrt(v64) / math.sqrt(1 - b264 ** st) + eps64)
    # |p| ~ 0.02-0.06 (fp32 ulp 2-4e-9); 5 steps of rounding stay within a few ulp
    np.testing.assert_allclose(p, p64, rtol=1e-6, atol=3e-8)
    np.testing.assert_allclose(m, m64, rtol=1e-5, atol=1e-12)
    np.testing.assert_allclose(v, v64, rtol=1e-5, atol=1e-18)


# ---------------------------------------------------------------------------
# conversions, norm, clip coefficient
# ---------------------------------------------------------------------------

def _special_f32():
    vals = [0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 3.4028235e38, -3.4028235e38, 1e-45, -1e-45,
            1.17549435e-38, 65504.0, 65519.996, 65520.0, 65536.0, 5.96e-8, 2.98e-8, 2.9802322e-08,
            1.0000001, 1.00390625, 1.0078125, 1.01171875]
    u = np.array(vals, dtype=np.float32).view(np.uint32)
    # exact bf16 ties (low half == 0x8000) at even and odd bf16 LSB, and neighbours
    ties = np.array([0x3f808000, 0x3f818000, 0x3f807fff, 0x3f808001, 0x7f7f8000, 0x7f7fffff,
                     0x00008000, 0x00018000, 0x80008000], dtype=np.uint32)
    return np.concatenate([u, ties]).view(np.float32)


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(11)
    bits = rng.integers(0, 2**32, size=1 << 22, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([bits.view(np.float32), _special_f32()])
    ours = O.f32_to_bf16(x)
    theirs = torch.from_numpy(x.copy()).bfloat16().view(torch.int16).numpy().view(np.uint16)
    finite = ~np.isnan(x)
    assert np.array_equal(ours[finite], theirs[finite])
    assert (ours[~finite] == 0x7FC0).all()  # simd.h:82


def test_f16_rne_matches_numpy():
    rng = np.random.default_rng(12)
    bits = rng.integers(0, 2**32, size=1 << 18, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([bits.view(np.float32), _special_f32(),
                        rng.normal(0, 1e-5, 1 << 16).astype(np.float32)])
    lib = O.lib()
    ours = np.array([lib.orc_f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    with np.errstate(over="ignore"):
        theirs = x.astype(np.float16).view(np.uint16)
    finite = ~np.isnan(x)
    assert np.array_equal(ours[finite], theirs[finite])
    back = np.array([lib.orc_f16_to_f32(int(h)) for h in ours[finite][:4096]], dtype=np.float32)
    assert np.array_equal(back, ours[finite][:4096].view(np.float16).astype(np.float32))


@pytest.mark.parametrize("n", [100001, 3_000_017])
def test_sqnorm_is_exact_float64_sum(n):
    # 3 M elements take the blocked parallel path; outliers x100 and a wide
    # dynamic range make plain float64 accumulation visibly inexact
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1e-3, n).astype(np.float32)
    x[rng.integers(0, n, n // 1000)] *= 100
    x[: n // 7] *= 1e-6
    g = torch.from_numpy(x).bfloat16()
    gb = _np_bits(g, "bf16")
    got = O.grad_sqnorm(gb, "bf16")
    exact = math.fsum(float(v) * float(v) for v in g.float().numpy())
    assert abs(got - exact) <= 1e-15 * exact
    # the same value in fp32 and fp16 storage
    assert abs(O.grad_sqnorm(g.float().numpy().copy()) - exact) <= 1e-15 * exact


@pytest.mark.parametrize("n", [5, 100001, 3_000_017])
def test_sqnorm_of_non_finite_grads(n):
    """An inf grad gives inf, as math.fsum and torch's norm do (the
    compensation term must not turn inf - inf into NaN); a NaN grad gives NaN.
    Both the short and the blocked parallel path.  Finite float32 grads cannot
    overflow the float64 sum: each square is at most 1.2e77."""
    x = np.full(n, 1e-3, np.float32)
    for pos in (0, n // 2, n - 1):
        y = x.copy()
        y[pos] = np.inf
        assert O.grad_sqnorm(y) == math.inf
        assert O.grad_sqnorm(y.astype(np.float16).view(np.uint16), "f16") == math.inf
        y[pos] = -np.inf
        assert O.grad_sqnorm(y) == math.inf
        y[pos] = np.nan
        assert math.isnan(O.grad_sqnorm(y))
    big = np.full(n, np.finfo(np.float32).max, np.float32)
    exact = math.fsum([float(big[0]) ** 2] * n)
    assert abs(O.grad_sqnorm(big) - exact) <= 1e-15 * exact
    assert math.fsum([math.inf, 1.0]) == math.inf


def test_clip_coef_matches_torch_clip_grad_norm():
    rng = np.random.default_rng(6)
    for scale, max_norm in ((1e-3, 1.0), (1e-1, 1.0), (1e-5, 1.0), (1.0, 0.5)):
        g = torch.from_numpy(rng.normal(0, scale, 50000).astype(np.float32))
        sq = O.grad_sqnorm(g.numpy().copy())
        coef, norm = O.clip_coef(sq, max_norm)
        w = torch.nn.Parameter(torch.zeros_like(g))
        w.grad = g.clone()
        total = torch.nn.utils.clip_grad_norm_([w], max_norm)
        assert abs(float(total) - norm) <= 2e-7 * norm
        expected = g * min(1.0, max_norm / (float(total) + 1e-6))
        torch.testing.assert_close(torch.from_numpy(g.numpy() * np.float32(coef)), expected,
                                   rtol=2e-7, atol=0)
        torch.testing.assert_close(w.grad, expected, rtol=2e-7, atol=0)


GPT2_SIZES = [768, 768, 768 * 2304, 2304, 768 * 768, 768, 768, 768, 768 * 3072, 3072, 3072 * 768, 768]


@pytest.mark.parametrize("per_tensor", [False, True])
def test_c1_gpt2_block_full_size_vs_compiled_reference(per_tensor):
    """Config C1 on the CPU: the GPT-2-small block (7,087,872 params), 10 steps,
    lr 1e-5, wd 0.01, fresh grads per step (seed 1000 + step), as one flat
    step_chunk call or as one call per tensor (step / step_with_grad_views,
    layer_adam.py:299-327).  Oracle == compiled reference, bit for bit."""
    ref = _ref_or_skip()
    n = sum(GPT2_SIZES)
    assert n == 7_087_872
    p0 = np.random.default_rng(1).normal(0, 0.02, n).astype(np.float32)
    p = torch.from_numpy(p0.copy())
    m, v = torch.zeros(n), torch.zeros(n)
    pb, mb, vb = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    ref.create_adam(0, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, False)
    opt = O.OracleAdam(1e-5, (0.9, 0.999), 1e-8, 0.01, True)
    bounds = np.cumsum([0] + GPT2_SIZES) if per_tensor else np.array([0, n])
    for step in range(1, 11):
        g = torch.from_numpy(np.random.default_rng(1000 + step).normal(0, 1e-3, n).astype(np.float32)).bfloat16()
        gb = _np_bits(g, "bf16")
        for lo, hi in zip(bounds[:-1], bounds[1:]):
            ref.adam_update(0, step, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, p[lo:hi], g[lo:hi], m[lo:hi], v[lo:hi])
            opt.update(step, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, pb[lo:hi], gb[lo:hi], mb[lo:hi], vb[lo:hi],
                       g16="bf16")
    assert np.array_equal(p.numpy().view(np.uint32), pb.view(np.uint32))
    assert np.array_equal(m.numpy().view(np.uint32), mb.view(np.uint32))
    assert np.array_equal(v.numpy().view(np.uint32), vb.view(np.uint32))
