"""CPU checks of the C-ABI library: it loads, exports every declared symbol,
and its host-side logic (the beta-power state machine, argument validation,
workspace sizing) is right.  No kernel is launched here."""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest

from oracle import oracle as O
from slideformer_amd import _lib

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "layer_adam.h")


def _read(path, mode="r"):
    with open(path, mode) as f:
        return f.read()


def declared_functions():
    text = _read(HEADER)
    return sorted(set(re.findall(r"^\s*(?:int|uint64_t|const char\*)\s+(la_\w+)\s*\(", text, re.M)))


def test_header_and_binding_agree():
    assert declared_functions() == sorted(_lib.EXPORTED)


def test_library_exports_every_declared_symbol():
    L = _lib.load()
    for name in declared_functions():
        assert hasattr(L, name), name
    version = int(re.search(r"#define LA_ABI_VERSION (\d+)", _read(HEADER)).group(1))
    assert L.la_abi_version() == version == _lib.ABI_VERSION == 9
    header = _read(HEADER)
    for name in ("LA_OK", "LA_EINVAL", "LA_EDTYPE", "LA_ENOMEM", "LA_ERANGE", "LA_EFAULT", "LA_F32", "LA_BF16", "LA_F16", "LA_ON_HOST_P",
                 "LA_ON_HOST_M", "LA_ON_HOST_V", "LA_ON_HOST_G", "LA_ON_HOST_OUT", "LA_ON_HOST_ALL",
                 "LA_NORM_MULTI_MAX"):
        value = int(re.search(rf"#define {name} \(?(-?\d+)u?\)?", header).group(1))
        assert getattr(_lib, name) == value, name


def test_library_is_gfx950_code_object():
    # the fat binary embeds an amdgcn code object for gfx950 only
    blob = _read(_lib.LIB_PATH, "rb")
    assert b"gfx950" in blob
    for other in (b"gfx942", b"gfx90a", b"gfx1100"):
        assert other not in blob


def _scalars(L, id_, *args):
    sc = _lib.LaScalars()
    assert L.la_scalars(id_, *args, ctypes.byref(sc)) == 0
    return sc


@pytest.mark.parametrize("betas", [(0.9, 0.999), (0.8, 0.95)])
def test_host_state_machine_matches_oracle(betas):
    """la_scalars replays IncrementStep/update_state (cpu_adam.h:57-89) bit for bit:
    multiply path, pow path (several calls per step), step jumps, beta changes,
    bias_correction off, lr/wd changes."""
    L = _lib.load()
    b1, b2 = betas
    L.la_create(901, 1e-3, b1, b2, 1e-8, 0.01, 1, 0)
    orc = O.OracleAdam(1e-3, betas, 1e-8, 0.01, True)
    seq = []
    for st in range(1, 120):
        seq.append((st, 1e-3, b1, b2, 1e-8, 0.01, 1))
        if st % 7 == 0:
            seq.append((st, 1e-3, b1, b2, 1e-8, 0.01, 1))          # second chunk: pow path
    seq += [(500, 2e-4, b1, b2, 1e-6, 0.1, 1), (501, 2e-4, b1, b2, 1e-6, 0.1, 0),
            (502, 2e-4, 0.85, b2, 1e-6, 0.1, 1), (503, 2e-4, 0.85, b2, 1e-6, 0.0, 1),
            (1, 1e-3, b1, b2, 1e-8, 0.01, 1)]
    lib = O.lib()
    for (st, lr, bb1, bb2, eps, wd, bc) in seq:
        sc = _scalars(L, 901, st, lr, bb1, bb2, eps, wd, bc)
        lib.orc_increment_step(orc.s, st, bb1, bb2)
        lib.orc_update_state(orc.s, lr, eps, wd, bc)
        ref = orc.scalars()  # b1t, b2t, bc1, bc2, step_size, w_decay, 1-b1, 1-b2
        got = np.array([sc.beta1_t, sc.beta2_t, sc.bias_correction1, sc.bias_correction2,
                        sc.step_size, sc.w_decay, sc.one_minus_beta1, sc.one_minus_beta2],
                       dtype=np.float32)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (st, got, ref)
        assert sc.step == orc.s.step
        assert sc.decay_mode == (0 if np.float32(wd) <= 0 else 2)
    L.la_destroy(901)


def test_l2_mode_flag():
    L = _lib.load()
    L.la_create(902, 1e-3, 0.9, 0.999, 1e-8, 0.1, 0, 0)
    sc = _scalars(L, 902, 1, 1e-3, 0.9, 0.999, 1e-8, 0.1, 1)
    assert sc.decay_mode == 1 and sc.weight_decay == np.float32(0.1)
    L.la_destroy(902)


def test_error_codes_without_launch():
    L = _lib.load()
    sc = _lib.LaScalars()
    # unknown id
    assert L.la_scalars(123456, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1, ctypes.byref(sc)) == _lib.LA_EINVAL
    assert L.la_adam_update(123456, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1, 0, None, 1, None, 0, None, None,
                            10, None, None, None) == _lib.LA_EINVAL
    # unregistered dtype triples (cpu_adam_impl.cpp:181-189) and unknown codes
    for trip in [(0, 0, 1), (1, 2, 0), (2, 1, 0), (1, 1, 2), (0, 1, 2), (7, 0, 0)]:
        assert L.la_adamw_step(ctypes.byref(sc), trip[0], None, trip[1], None, trip[2], None, None, 10,
                               None, None, None) == _lib.LA_EDTYPE
    # n == 0 is a no-op (the reference test registers an empty layer)
    assert L.la_adamw_step(ctypes.byref(sc), 0, None, 1, None, 0, None, None, 0, None, None, None) == 0
    # null buffers with n > 0
    assert L.la_adamw_step(ctypes.byref(sc), 0, None, 1, None, 0, None, None, 5, None, None, None) == _lib.LA_EINVAL
    # misaligned element pointers (odd address for a 4-byte type)
    assert L.la_adamw_step(ctypes.byref(sc), 0, 0x1001, 1, 0x2000, 0, 0x3000, 0x4000, 5, None, None,
                           None) == _lib.LA_EINVAL
    assert L.la_grad_sqnorm(1, None, 10, None, 0, None, 0, None) == _lib.LA_EINVAL
    assert L.la_grad_norm_clip(1, None, 10, None, 0, None, 0, 1.0, None, None, None) == _lib.LA_EINVAL
    assert L.la_clip_coef(None, 1.0, None, None, None) == _lib.LA_EINVAL
    # the no-allocation norm checks coef before it looks anything up on a device
    assert L.la_grad_norm_clip_noalloc(1, None, 10, None, 0, 1.0, None, None, None) == _lib.LA_EINVAL
    assert b"scratch" in L.la_strerror(_lib.LA_ERANGE)
    # aligned host memory handed to the device entry points: refused before any launch
    host = np.zeros(64, np.float32)
    hp = host.ctypes.data + (-host.ctypes.data) % 16
    assert L.la_adamw_step(ctypes.byref(sc), 0, hp, 0, hp, 0, hp, hp, 8, None, None, None) == _lib.LA_EFAULT
    assert L.la_grad_sqnorm(0, hp, 8, hp, 64, hp, 0, None) == _lib.LA_EFAULT
    assert L.la_clip_coef(hp, 1.0, hp, None, None) == _lib.LA_EFAULT
    # the multi-buffer norm: buffer count, null / misaligned buffers, workspace size,
    # host memory; every check comes before the first launch
    bufs = (_lib.LaGradBuffer * 33)()
    for b in bufs:
        b.g, b.n = hp, 8
    multi = L.la_grad_norm_multi
    assert multi(1, None, 1, hp, 64, hp, 0, 1.0, hp, None, None) == _lib.LA_EINVAL
    assert multi(1, bufs, 0, hp, 64, hp, 0, 1.0, hp, None, None) == _lib.LA_EINVAL
    assert multi(1, bufs, _lib.LA_NORM_MULTI_MAX + 1, hp, 64, hp, 0, 1.0, hp, None, None) == _lib.LA_EINVAL
    assert multi(7, bufs, 1, hp, 64, hp, 0, 1.0, hp, None, None) == _lib.LA_EDTYPE
    assert multi(1, bufs, 2, hp, 64, None, 0, 1.0, hp, None, None) == _lib.LA_EINVAL
    assert multi(1, bufs, 2, hp + 4, 64, hp, 0, 1.0, hp, None, None) == _lib.LA_EINVAL    # workspace alignment
    assert multi(1, bufs, 2, hp, 0, hp, 0, 1.0, hp, None, None) == _lib.LA_EINVAL         # workspace too small
    bufs[1].g = hp + 1                                                                    # odd for 2-byte grads
    assert multi(1, bufs, 2, hp, 64, hp, 0, 1.0, hp, None, None) == _lib.LA_EINVAL
    bufs[1].g, bufs[1].n = None, 5
    assert multi(1, bufs, 2, hp, 64, hp, 0, 1.0, hp, None, None) == _lib.LA_EINVAL
    bufs[1].n = 0                                                                         # empty: g may be NULL
    assert multi(1, bufs, 2, hp, 64, hp, 0, 1.0, hp, None, None) == _lib.LA_EFAULT
    assert multi(1, bufs, _lib.LA_NORM_MULTI_MAX, hp, 64, hp, 1, 0.0, None, None, None) == _lib.LA_EFAULT
    assert b"device memory" in L.la_strerror(_lib.LA_EFAULT)
    assert b"dtype" in L.la_strerror(_lib.LA_EDTYPE)
    assert b"memory" in L.la_strerror(_lib.LA_ENOMEM)


def test_grad_sqnorm_workspace_is_bounded():
    """one float64 partial per stage-1 workgroup; the grid is capped so the
    folding workgroup reads a bounded number of partials."""
    L = _lib.load()
    sizes = (0, 1, 7, 4096, 4097, 8 * 256 * 3, 10**6, 218_112_000, 1 << 40)
    ws = [L.la_grad_sqnorm_workspace(n) for n in sizes]
    assert ws[0] == ws[1] == 8                      # one workgroup
    assert all(w % 8 == 0 and w >= 8 for w in ws)
    assert ws == sorted(ws)                         # non-decreasing in n
    assert ws[-1] == L.la_grad_sqnorm_workspace(1 << 35) <= 64 * 1024   # capped


def _segments(specs):
    segs = (_lib.LaSegment * len(specs))()
    for k, (p, g, m, v, out, n) in enumerate(specs):
        segs[k].p, segs[k].g, segs[k].m, segs[k].v, segs[k].p_bf16_out, segs[k].n = p, g, m, v, out, n
    return segs


def test_multi_update_host_logic_without_launch():
    """la_adam_update_multi: argument checks come before any state change, and
    the beta-power state advances once per segment, n = 0 segments included,
    exactly as the same number of la_adam_update calls would."""
    L = _lib.load()
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    lib = O.lib()
    L.la_create(904, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1, 0)
    replay = []

    def scalars(step):
        sc = _scalars(L, 904, step, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1)
        replay.append(step)
        return sc

    for st in range(1, 5):
        scalars(st)
    args = (904, 5, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1, 0, 1, 0)
    assert L.la_adam_update_multi(*args, None, -1, None, None) == _lib.LA_EINVAL
    assert L.la_adam_update_multi(*args, None, 2, None, None) == _lib.LA_EINVAL
    # a misaligned pointer: rejected, nothing advanced
    bad = _segments([(0x1001, 0x2000, 0x3000, 0x4000, None, 8)])
    assert L.la_adam_update_multi(*args, bad, 1, None, None) == _lib.LA_EINVAL
    # aligned addresses that are not device memory (no GPU here, or host
    # memory on a GPU box) in the second segment: rejected, nothing advanced
    host = np.zeros(64, np.float32)
    hp = host.ctypes.data + (-host.ctypes.data) % 16
    bad = _segments([(None,) * 5 + (0,), (hp, hp, hp, hp, None, 4)])
    assert L.la_adam_update_multi(*args, bad, 2, None, None) == _lib.LA_EFAULT
    # unknown id: nothing to advance
    assert L.la_adam_update_multi(123457, *args[1:], _segments([(None,) * 5 + (0,)]), 1, None, None) == _lib.LA_EINVAL
    # three empty segments: no launch, three state advances
    assert L.la_adam_update_multi(*args, _segments([(None,) * 5 + (0,)] * 3), 3, None, None) == 0
    replay += [5, 5, 5]
    # an unregistered triple advances the state once, then fails like the first separate call
    assert L.la_adam_update_multi(904, 6, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1, 0, 0, 1,
                                  _segments([(None,) * 5 + (0,)] * 2), 2, None, None) == _lib.LA_EDTYPE
    replay += [6]
    got = scalars(7)
    for st in replay:
        lib.orc_increment_step(orc.s, st, 0.9, 0.999)
        lib.orc_update_state(orc.s, 1e-3, 1e-8, 0.01, 1)
    ref = orc.scalars()
    vals = np.array([got.beta1_t, got.beta2_t, got.bias_correction1, got.bias_correction2, got.step_size,
                     got.w_decay, got.one_minus_beta1, got.one_minus_beta2], dtype=np.float32)
    assert np.array_equal(vals.view(np.uint32), ref.view(np.uint32))
    assert got.step == orc.s.step == 7
    L.la_destroy(904)


def test_pipeline_workspace_follows_the_placement():
    """la_pipeline_workspace_bytes holds one 256-byte aligned region per
    host-resident array and slot (chunk rounded down to 16 elements); device
    arrays take no staging; unknown placement bits give 0."""
    L = _lib.load()
    F32, BF16 = _lib.LA_F32, _lib.LA_BF16
    P, M, V, G, OUT = (_lib.LA_ON_HOST_P, _lib.LA_ON_HOST_M, _lib.LA_ON_HOST_V, _lib.LA_ON_HOST_G,
                       _lib.LA_ON_HOST_OUT)
    f32_region, bf16_region = 4096, 2048     # 992 elements: 3968 B and 1984 B, rounded up to 256
    cases = {P | M | V: 3 * f32_region, P | M | V | G | OUT: 3 * f32_region + 2 * bf16_region,
             P | G: f32_region + bf16_region, M | V: 2 * f32_region, G: bf16_region, OUT: bf16_region, 0: 0}
    for mask, per_slot in cases.items():
        assert L.la_pipeline_workspace_bytes(1000, 2, F32, BF16, F32, mask) == 2 * per_slot, mask
    assert L.la_pipeline_workspace_bytes(1000, 2, F32, BF16, F32, _lib.LA_ON_HOST_ALL | 32) == 0
    assert L.la_pipeline_workspace_bytes(15, 2, F32, BF16, F32, P) == 0


def test_segment_layout_is_six_words():
    """LayerAdam builds la_segment_t arrays as six uint64 per segment
    (p, g, m, v, p_bf16_out, n); the struct must have exactly that layout."""
    S = _lib.LaSegment
    assert ctypes.sizeof(S) == 48
    assert [getattr(S, f).offset for f in ("p", "g", "m", "v", "p_bf16_out", "n")] == [0, 8, 16, 24, 32, 40]
    header = _read(HEADER)
    body = re.search(r"typedef struct \{([^}]*)\} la_segment_t;", header).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    names = re.findall(r"(\w+);", body)
    assert names == ["p", "g", "m", "v", "p_bf16_out", "n"]


def test_state_machine_is_safe_under_concurrent_calls():
    """The beta-power state of one id is guarded by a mutex: 8 threads call
    la_scalars for the same step at once, 150 steps in a row (ctypes releases
    the GIL, so the calls really overlap).  Per step exactly one call takes the
    multiply path (the first one to hold the state) and the other seven the
    pow path (cpu_adam.h:57-89), each bit-exact with the oracle replaying that
    order; nothing tears."""
    import threading

    L = _lib.load()
    threads, steps = 8, 150
    L.la_create(905, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1, 0)
    barrier = threading.Barrier(threads)
    got = [[None] * steps for _ in range(threads)]

    def worker(t):
        for st in range(1, steps + 1):
            barrier.wait()
            sc = _scalars(L, 905, st, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1)
            got[t][st - 1] = (np.float32(sc.beta1_t), np.float32(sc.beta2_t), np.float32(sc.step_size),
                              np.float32(sc.bias_correction2), sc.step)

    ws = [threading.Thread(target=worker, args=(t,)) for t in range(threads)]
    for w in ws:
        w.start()
    for w in ws:
        w.join()
    L.la_destroy(905)
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    lib = O.lib()
    for st in range(1, steps + 1):
        expected = []
        for k in range(threads):                     # the order the lock admits them in
            lib.orc_increment_step(orc.s, st, 0.9, 0.999)
            lib.orc_update_state(orc.s, 1e-3, 1e-8, 0.01, 1)
            r = orc.scalars()
            expected.append((r[0], r[1], r[4], r[3], st))
        first, rest = expected[0], expected[1]
        assert all(e == rest for e in expected[1:])
        outs = [got[t][st - 1] for t in range(threads)]
        n_first = sum(o[:4] == first[:4] for o in outs)
        n_rest = sum(o[:4] == rest[:4] for o in outs)
        if first[:4] == rest[:4]:
            assert n_first == threads, st
        else:
            assert (n_first, n_rest) == (1, threads - 1), (st, outs, first, rest)
        assert all(o[4] == st for o in outs)


def test_header_is_usable_from_c(tmp_path):
    """tests/native/abi_from_c.c, compiled as C11 with -Wall -Werror against
    include/layer_adam.h and linked to the library, calls the host-side entry
    points; its beta-power scalars match the CPU checker bit for bit."""
    import os
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    src = os.path.join(os.path.dirname(__file__), "native", "abi_from_c.c")
    exe = str(tmp_path / "abi_from_c")
    libdir = os.path.dirname(_lib.LIB_PATH)
    subprocess.run([gcc, "-std=c11", "-Wall", "-Wextra", "-Werror", "-pedantic", "-I", os.path.dirname(HEADER),
                    src, "-L", libdir, "-lslideformer_amd", f"-Wl,-rpath,{libdir}", "-o", exe], check=True)
    res = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, (res.returncode, res.stderr)
    lines = res.stdout.split("\n")[:7]
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    lib = O.lib()
    for st, line in zip((1, 2, 3, 4, 5, 5, 9), lines):
        lib.orc_increment_step(orc.s, st, 0.9, 0.999)
        lib.orc_update_state(orc.s, 1e-3, 1e-8, 0.01, 1)
        r = orc.scalars()    # b1t, b2t, bc1, bc2, step_size, w_decay, ...
        f = line.split()
        assert int(f[0]) == st
        got = np.array([float.fromhex(x) for x in f[1:7]], dtype=np.float32)
        assert np.array_equal(got.view(np.uint32), r[:6].view(np.uint32)), (st, got, r[:6])
        assert int(f[7]) == 2


def test_library_of_another_abi_version_is_refused(tmp_path):
    """A library built from other sources (here a stand-in that only reports ABI
    version 1) is refused at load with a message to rebuild, before any of its
    symbols is bound."""
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    src = tmp_path / "old.c"
    src.write_text("int la_abi_version(void) { return 1; }\n")
    so = tmp_path / "libold.so"
    subprocess.run([gcc, "-shared", "-fPIC", "-o", str(so), str(src)], check=True)
    saved = _lib._lib
    _lib._lib = None
    try:
        with pytest.raises(ImportError, match="C-ABI version 1"):
            _lib.load(str(so))
    finally:
        _lib._lib = saved


def _header_prototypes():
    """{name: (return kind, [parameter kinds])} of every function include/layer_adam.h declares.
    Kinds: ptr, f32, f64, i32, u32, u64."""
    text = re.sub(r"/\*.*?\*/", "", _read(HEADER), flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    scalar = {"float": "f32", "double": "f64", "int": "i32", "int32_t": "i32", "unsigned": "u32",
              "uint32_t": "u32", "uint64_t": "u64", "la_stream_t": "ptr"}

    def kind(decl):
        decl = decl.strip()
        if "*" in decl:
            return "ptr"
        words = [w for w in decl.split() if w != "const"]
        return scalar[words[0]]

    out = {}
    for ret, name, params in re.findall(r"^\s*(int|uint64_t|const char\*)\s+(la_\w+)\s*\(([^)]*)\)\s*;", text,
                                        re.M | re.S):
        params = [] if params.strip() == "void" else [kind(p) for p in params.split(",")]
        out[name] = (kind(ret), params)
    return out


def _ctypes_kind(t):
    if t in (ctypes.c_void_p, ctypes.c_char_p) or (isinstance(t, type) and issubclass(t, ctypes._Pointer)):
        return "ptr"
    return {ctypes.c_float: "f32", ctypes.c_double: "f64", ctypes.c_int: "i32", ctypes.c_uint: "u32",
            ctypes.c_uint64: "u64"}[t]


def test_binding_argtypes_follow_the_header():
    """Every ctypes prototype of _lib (argument and return types) is the
    header's, kind by kind: pointers, 32-bit ints, unsigned, 64-bit sizes and
    floats in the same positions."""
    L = _lib.load()
    protos = _header_prototypes()
    assert sorted(protos) == sorted(_lib.EXPORTED)
    for name, (ret, params) in protos.items():
        fn = getattr(L, name)
        assert [_ctypes_kind(t) for t in fn.argtypes] == params, name
        assert _ctypes_kind(fn.restype) == ret, name


def test_struct_mirrors_match_the_c_layout(tmp_path):
    """The ctypes mirrors of la_scalars_t, la_segment_t, la_grad_buffer_t and
    la_pipeline_stats_t have the C compiler's size, field offsets and field
    sizes (a C program built against the header prints them)."""
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    mirrors = {"la_scalars_t": _lib.LaScalars, "la_segment_t": _lib.LaSegment,
               "la_grad_buffer_t": _lib.LaGradBuffer, "la_pipeline_stats_t": _lib.LaPipelineStats}
    lines = ["#include <stddef.h>", "#include <stdio.h>", '#include "layer_adam.h"', "int main(void) {"]
    for cname, S in mirrors.items():
        lines.append(f'    printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in S._fields_:
            lines.append(f'    printf("{cname} {field} %zu %zu\\n", offsetof({cname}, {field}), '
                         f'sizeof((({cname}*)0)->{field}));')
    lines += ["    return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = str(tmp_path / "layout")
    subprocess.run([gcc, "-std=c11", "-Wall", "-Werror", "-I", os.path.dirname(HEADER), str(src), "-o", exe],
                   check=True)
    got = {}
    for line in subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split("\n"):
        if line:
            cname, field, *values = line.split()
            got[(cname, field)] = tuple(int(v) for v in values)
    for cname, S in mirrors.items():
        assert got[(cname, "size")] == (ctypes.sizeof(S),), cname
        for field, _ in S._fields_:
            desc = getattr(S, field)
            assert got[(cname, field)] == (desc.offset, desc.size), (cname, field)


@pytest.mark.parametrize("entry", ["LayerAdam", "cpu_adam_compat"])
def test_missing_library_fails_loudly(tmp_path, entry):
    """Without the built HIP library both entry points of the drop-in raise
    ImportError naming the build command: nothing falls back to a CPU path.
    Run in a fresh process pointed at a library file that does not exist."""
    import subprocess
    import sys

    code = {
        "LayerAdam": "from slideformer_amd import LayerAdam\nLayerAdam()\n",
        "cpu_adam_compat": ("from slideformer_amd import cpu_adam_compat\n"
                            "cpu_adam_compat.create_adam(0, 1e-3, 0.9, 0.999, 1e-8, 0.0, True, False)\n"),
    }[entry]
    env = dict(os.environ, SLIDEFORMER_AMD_LIB=str(tmp_path / "missing.so"))
    res = subprocess.run([sys.executable, "-c", code], env=env, cwd=REPO, capture_output=True, text=True,
                         timeout=600)
    assert res.returncode != 0
    assert "ImportError" in res.stderr and "there is no CPU fallback" in res.stderr, res.stderr[-2000:]
