"""CPU-only checks of the product library: it loads, exports every symbol of
include/lonnx.h, rejects calls before lx_init, and its host-side broadcast
planner addresses exactly the elements numpy broadcasting addresses.  Also
evaluates the device expf / erf restatements on the host against libm and the
oracle (tests/native/expf_check.cpp)."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import onnx_amd
from onnx_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lonnx.h")
NATIVE = os.path.join(ROOT, "tests", "native")


def header_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^[A-Za-z_][\w \*]*?\b(lx_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = L.lib()
    syms = header_symbols()
    assert len(syms) >= 25
    for s in syms:
        assert hasattr(lib, s), s
        assert s in L.SIGNATURES, f"{s} missing from the ctypes table"
    assert set(L.SIGNATURES) == set(syms)


def test_struct_layouts():
    assert ctypes.sizeof(L.LxTensor) == 4 + 4 + 8 * 8 + 8 + 8 + 4 + 4
    assert ctypes.sizeof(L.LxPlan) == 4 + 4 + 64 + 4 + 4 + 64 * 3 + 8


def test_calls_before_init_fail_cleanly():
    lib = L.lib()
    y = L.LxTensor()
    assert lib.lx_Add(None, None, ctypes.byref(y)) == L.ERR_NOT_INITIALIZED
    assert "lx_init" in L.last_error()
    assert lib.lx_dtype_size(L.FLOAT) == 4 and lib.lx_dtype_size(L.INT64) == 8 and lib.lx_dtype_size(8) == 0


def _offsets_from_plan(p, n):
    """Element offsets of A and B for every output element, from the collapsed plan."""
    dims = [p.dims[i] for i in range(p.rank)]
    idx = np.indices(dims).reshape(len(dims), -1)
    sa = np.array([p.a_strides[i] for i in range(p.rank)])[:, None]
    sb = np.array([p.b_strides[i] for i in range(p.rank)])[:, None]
    oa = (idx * sa).sum(0)
    ob = (idx * sb).sum(0)
    assert oa.size == n
    return oa, ob


def test_planner_matches_numpy_broadcasting():
    from oracle import oracle as O
    rng = np.random.default_rng(7)
    for _ in range(1500):
        ra, rb = (int(v) for v in rng.integers(0, 5, 2))
        a = tuple(int(v) for v in rng.choice([1, 2, 3, 4], ra))
        b = tuple(int(v) for v in rng.choice([1, 2, 3, 4], rb))
        st, p = L.plan_broadcast(a, b)
        exp = O.broadcast_shape(a, b)
        if exp is None:
            assert st == L.ERR_CANNOT_BROADCAST
            continue
        assert st == 0
        out = tuple(p.out_dims[i] for i in range(p.out_rank))
        assert out == exp
        n = int(np.prod(out)) if out else 1
        assert p.numel == n
        ia = np.broadcast_to(np.arange(int(np.prod(a)) if a else 1).reshape(a), out).reshape(-1)
        ib = np.broadcast_to(np.arange(int(np.prod(b)) if b else 1).reshape(b), out).reshape(-1)
        oa, ob = _offsets_from_plan(p, n)
        np.testing.assert_array_equal(oa, ia)
        np.testing.assert_array_equal(ob, ib)
        # innermost collapsed stride is 0 or 1 for both operands (kernel contract)
        assert p.a_strides[p.rank - 1] in (0, 1) and p.b_strides[p.rank - 1] in (0, 1)


@pytest.mark.parametrize("a,b,kind,dims,sa,sb", [
    ((1, 128, 384), (384,), L.PLAN_ND, (128, 384), (384, 1), (0, 1)),            # C1 bias
    ((1, 128, 384), (), L.PLAN_SCALAR_B, (49152,), (1,), (0,)),                  # C1 * 0.125
    ((8, 512, 768), (8, 512, 1), L.PLAN_ND, (4096, 768), (768, 1), (1, 0)),      # C2 x - mean
    ((16, 12, 512, 512), (16, 1, 1, 512), L.PLAN_ND, (16, 6144, 512), (3145728, 512, 1), (512, 0, 1)),  # C3
    ((64, 1, 4096), (1, 256, 4096), L.PLAN_ND, (64, 256, 4096), (4096, 0, 1), (0, 4096, 1)),           # C4
    ((32, 2048, 3072), (32, 2048, 3072), L.PLAN_SAME, (201326592,), (1,), (1,)),
])
def test_planner_config_shapes(a, b, kind, dims, sa, sb):
    st, p = L.plan_broadcast(a, b)
    assert st == 0 and p.kind == kind
    assert tuple(p.dims[i] for i in range(p.rank)) == dims
    assert tuple(p.a_strides[i] for i in range(p.rank)) == sa
    assert tuple(p.b_strides[i] for i in range(p.rank)) == sb


def _native():
    so = os.path.join(NATIVE, "libexpf_check.so")
    src = os.path.join(NATIVE, "expf_check.cpp")
    if not os.path.exists(so) or os.path.getmtime(so) < os.path.getmtime(src):
        subprocess.check_call(["/opt/rocm/bin/hipcc", "-O2", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
                               "--offload-host-only", "-x", "hip", "-fno-builtin", "-fopenmp", src, "-o", so])
    lib = ctypes.CDLL(so)
    lib.lx_test_expf_mismatches.restype = ctypes.c_longlong
    lib.lx_test_expf_mismatches.argtypes = [ctypes.c_uint64] * 3
    lib.lx_test_erf.restype = ctypes.c_float
    lib.lx_test_erf.argtypes = [ctypes.c_float]
    lib.lx_test_fastdiv.restype = ctypes.c_uint32
    lib.lx_test_fastdiv.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
    lib.lx_test_expf_core_range_mismatches.restype = ctypes.c_longlong
    lib.lx_test_expf_core_range_mismatches.argtypes = [ctypes.c_float, ctypes.c_float]
    for f in ("lx_test_expf_nonpos_mismatches", "lx_test_erf_fast_mismatches", "lx_test_gelu_mismatches"):
        getattr(lib, f).restype = ctypes.c_longlong
    lib.lx_test_sdiv32_mismatches.restype = ctypes.c_longlong
    lib.lx_test_sdiv32_mismatches.argtypes = [ctypes.c_double]
    return lib


def test_expf_method_matches_host_libm():
    """The device expf restatement equals the host expf (what MathF.Exp calls).
    Sampled here (every 61st bit pattern); LONNX_EXHAUSTIVE=1 checks all 2^32."""
    lib = _native()
    step = 1 if os.environ.get("LONNX_EXHAUSTIVE") == "1" else 61
    assert lib.lx_test_expf_mismatches(0, 1 << 32, step) == 0
    # dense sweep of the arguments Erf and Softmax produce: [-104, 0]
    lo = np.float32(-104.0).view(np.uint32)
    assert lib.lx_test_expf_mismatches(0x80000000, int(lo) + 1, 3) == 0


def test_device_erf_restatement_matches_oracle():
    from oracle import oracle as O
    lib = _native()
    xs = np.concatenate([np.linspace(-5, 5, 4001), [0.0, -0.0, 1e-6, -1e-6, 1e-30, 3.9, np.inf, -np.inf]])
    for v in xs.astype(np.float32):
        a, b = lib.lx_test_erf(float(v)), O.erf_f32(float(v))
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), v


def test_fastdiv():
    lib = _native()
    rng = np.random.default_rng(8)
    ds = [1, 2, 3, 5, 7, 12, 384, 512, 768, 4096, 6144, 65535, 65537, 1 << 20, 1000003, (1 << 31) - 1, 1 << 31]
    ds += [int(v) for v in rng.integers(1, 1 << 31, 50)]
    for d in ds:
        ns = [0, 1, d - 1, d, d + 1, (1 << 31) - 1] + [int(v) for v in rng.integers(0, 1 << 31, 200)]
        for n in ns:
            if 0 <= n < (1 << 31):
                assert lib.lx_test_fastdiv(n, d) == n // d, (n, d)


def test_expf_core_equals_host_expf_on_its_whole_range():
    """The early-out-free expf core (Horner form of the polynomial, where the published routine splits it)
    returns the host expf's bits for every float in [-104, 88], by exhaustion."""
    assert _native().lx_test_expf_core_range_mismatches(-104.0, 88.0) == 0


def test_division_free_sequences_are_exact():
    """The device Erf / GELU replace IEEE divisions and the expf early-outs by
    exact equivalents; each is proven here by exhaustion on the host:
      x / 1.4142135f  == fma(x, zh, x * zl) (zh + zl = 1/1.4142135f split into two
                         floats) for every x with |x| >= 2^-100; below, a quotient
                         near the denormal range can be one ulp off (some are: the
                         check sees them), which the GELU element's own exhaustive
                         check shows its output never depends on
      1 / d           == one float Newton step from the correctly rounded seed
                         for every float d in [1, 2^126); from a seed one ulp
                         off it fails at exactly 33 significands per binade
                         (the device check shows v_rcp_f32 never lands there)
      expf(x)         == the clamped early-out-free expf for every x <= 0."""
    lib = _native()
    div = (ctypes.c_longlong * 2)()
    lib.lx_test_div_sqrt2_mismatches(div)
    assert div[0] == 0
    assert div[1] > 0
    out = (ctypes.c_longlong * 2)()
    lib.lx_test_recip_mismatches(out)
    assert out[0] == 0
    assert out[1] == 33 * 126
    assert lib.lx_test_expf_nonpos_mismatches() == 0


def test_branch_free_erf_equals_reference_formula():
    """The device Erf core (clamped reciprocal argument, early-out-free expf)
    returns the A&S 7.1.26 formula's bits for all 2^32 inputs."""
    lib = _native()
    assert lib.lx_test_erf_fast_mismatches() == 0


def test_fused_gelu_equals_unfused_chain():
    """The fused GELU element (sign copied onto erf, max-clamped exponential
    argument) returns the unfused five-node chain's bits for all 2^32 inputs."""
    lib = _native()
    assert lib.lx_test_gelu_mismatches() == 0


@pytest.mark.parametrize("rel", [0.0, 2.0 ** -21, -(2.0 ** -21)])
def test_integer_division_by_double_reciprocal(rel):
    """The device int32 quotient (sdiv32_core: double reciprocal from a seed,
    one Newton step, trunc((a + sign(a) 0.5) * y)) equals C integer division for
    every divisor magnitude up to 2^20 and 2^22 random larger ones, at the
    dividends next to multiples of the divisor with every sign, all a, b in
    [-2^10, 2^10) and the extreme values -- from an exact seed and from seeds
    off by 2^-21 either way (the device seed is within 2^-21: see
    test_device_rcp_f32_error_bound)."""
    assert _native().lx_test_sdiv32_mismatches(rel) == 0


def test_integer_division_check_detects_a_weak_seed():
    """The same check fails when the seed is too coarse for one Newton step (2^-8 off):
    the check can see a wrong quotient."""
    assert _native().lx_test_sdiv32_mismatches(2.0 ** -8) > 0
