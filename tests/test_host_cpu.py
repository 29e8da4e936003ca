"""Host-side checks that need no GPU: the C ABI library loads and exports
every symbol of include/msda_hip.h, rejects bad arguments before touching
the device, the Python boundary validates like the reference
(src/msda_triton/ops.py:140-184, tests/test_msda.py:253-269), and the
benchmark presets carry the published sizes and byte counts."""

import ctypes
import re
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from msda_cases import make_inputs
from msda_triton_amd import _native, multi_scale_deformable_attention, presets

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "msda_hip.h"


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(msda_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _native.load()


def test_library_exports_every_declared_symbol(lib):
    names = header_functions()
    assert names == sorted(_native.SIGNATURES), names
    for name in names:
        assert hasattr(lib, name), name
    syms = subprocess.run(["nm", "-D", "--defined-only", str(_native.LIB_PATH)],
                          capture_output=True, text=True, check=True).stdout
    for name in names:
        assert re.search(rf"\bT {name}$", syms, re.M), name


def test_abi_version_and_error_strings(lib):
    assert lib.msda_abi_version() == (1 << 16) | 5
    for code in range(5):
        assert lib.msda_error_string(code)
    assert b"unknown" in lib.msda_error_string(99)


FWD_ARGS = dict(value=1, shapes=1, starts=1, loc=1, attn=1, out=1,
                B=2, S=10, M=2, D=8, Q=3, L=1, K=2, dtype=0)


def call_fwd(lib, **kw):
    a = dict(FWD_ARGS, **kw)
    return lib.msda_forward(a["value"], a["shapes"], a["starts"], a["loc"], a["attn"], a["out"],
                            a["B"], a["S"], a["M"], a["D"], a["Q"], a["L"], a["K"], a["dtype"], None)


def call_bwd(lib, **kw):
    a = dict(FWD_ARGS, gout=1, gv=1, acc=None, gl=1, ga=1)
    a.update(kw)
    return lib.msda_backward(a["value"], a["shapes"], a["starts"], a["loc"], a["attn"], a["gout"],
                             a["gv"], a["acc"], a["gl"], a["ga"], a["B"], a["S"], a["M"], a["D"],
                             a["Q"], a["L"], a["K"], a["dtype"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(dtype=7), 2),
    (dict(B=-1), 1),
    (dict(K=-3), 1),
    (dict(L=65), 3),
    (dict(D=1000), 3),            # fp32 row of 4000 bytes: wider than one wave
    (dict(out=None), 1),
    (dict(loc=None), 1),
    (dict(shapes=None), 1),
    (dict(B=0), 0),               # empty: nothing to launch
    (dict(Q=0), 0),
])
def test_forward_argument_errors_return_before_any_launch(lib, kw, code):
    assert call_fwd(lib, **kw) == code


@pytest.mark.parametrize("kw,code", [
    (dict(dtype=3), 2),
    (dict(gl=None), 1),
    (dict(gout=None), 1),
    (dict(gv=None), 1),
    (dict(L=100), 3),
    (dict(B=0, S=0, Q=0), 0),     # nothing to zero, nothing to launch
])
def test_backward_argument_errors_return_before_any_launch(lib, kw, code):
    assert call_bwd(lib, **kw) == code


def test_missing_library_raises_at_call_time(monkeypatch, tmp_path):
    monkeypatch.setattr(_native, "LIB_PATH", tmp_path / "nope.so")
    monkeypatch.setattr(_native, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        _native.load()


def test_check_raises_runtime_error_with_message():
    with pytest.raises(RuntimeError, match="unsupported dtype"):
        _native.check(2, "msda_forward")


# --- Python boundary validation (reference: tests/test_msda.py:253-269) ---

def _inputs():
    return make_inputs(B=1, Q=8, M=2, D=16, shapes=[(6, 6)], K=2, dtype=torch.float32, device="cpu")


def test_rejects_mismatched_shapes_and_dtypes():
    value, shapes, starts, loc, attn = _inputs()
    with pytest.raises(ValueError, match="attention_weights"):
        multi_scale_deformable_attention(value, shapes, starts, loc, attn[:, :, :, :, :1])
    with pytest.raises(ValueError, match="dtypes"):
        multi_scale_deformable_attention(value, shapes, starts, loc.half(), attn)
    with pytest.raises(ValueError, match="CUDA"):
        multi_scale_deformable_attention(value, shapes, starts, loc, attn)


@pytest.mark.parametrize("mutate,match", [
    (lambda v, s, st, l, a: (v[0], s, st, l, a), "value must be"),
    (lambda v, s, st, l, a: (v, s, st, l[..., :1], a), "sampling_locations must be"),
    (lambda v, s, st, l, a: (v, s, st, l[:, :, :1], a[:, :, :1]), "inconsistent"),
    (lambda v, s, st, l, a: (v, s[:, :1], st, l, a), "spatial_shapes"),
    (lambda v, s, st, l, a: (v.double(), s, st, l.double(), a.double()), "unsupported dtype"),
])
def test_validation_messages(mutate, match):
    args = mutate(*_inputs())
    with pytest.raises(ValueError, match=match):
        multi_scale_deformable_attention(*args)


# --- Presets: published sizes and the reference's byte accounting ---------

@pytest.mark.parametrize("name,S,Q,fwd,bwd", [
    ("tiny", 1360, 100, 6_809_600, 13_516_800),
    ("decoder", 22223, 300, 40_857_600, 81_100_800),
    ("high_contention", 22223, 300, 40_857_600, 81_100_800),
    ("encoder", 22223, 22223, 1_513_297_408, 3_003_838_464),
    ("mask2former_fp32", 21504, 21504, 2_207_514_624, 4_370_989_056),
    ("mask2former_bf16", 21504, 21504, 1_103_757_312, 2_185_494_528),
])
def test_preset_sizes_and_bytes(name, S, Q, fwd, bwd):
    c = presets.preset_dims(name)
    assert (c["S"], c["Q"]) == (S, Q)
    assert presets.algorithmic_bytes(name) == (fwd, bwd)


def test_decoder_pyramid_matches_reference_shapes():
    assert presets.pyramid(800, 1333) == [(100, 167), (50, 84), (25, 42), (13, 21)]
    assert presets.pyramid(1024, 1024, 3) == [(128, 128), (64, 64), (32, 32)]


def test_preset_inputs_are_seeded_and_rounded():
    a = presets.make_preset_inputs("tiny")
    b = presets.make_preset_inputs("tiny")
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    value, shapes, starts, loc, attn = presets.make_preset_inputs("decoder")
    assert value.dtype == loc.dtype == attn.dtype == torch.bfloat16
    assert starts.tolist() == [0, 16700, 20900, 21950]
    torch.testing.assert_close(attn.float().sum((-1, -2)), torch.ones(4, 300, 8), atol=2e-2, rtol=0)
    _, _, _, loc_e, _ = presets.make_preset_inputs("encoder")
    assert loc_e.min() >= -0.1 and loc_e.max() <= 1.1


def test_bench_refuses_more_than_one_gpu():
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=60)
    assert res.returncode == 2 and "one GPU" in res.stderr


def test_graft_entry_points_exist():
    sys.path.insert(0, str(ROOT))
    import __graft_entry__ as ge

    assert callable(ge.build) and callable(ge.smoke)


# --- torch.library registration and call-site shims (CPU: fake tensors) ---

def test_custom_ops_are_registered_with_fake_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    import msda_triton_amd

    assert callable(msda_triton_amd.msda_op)
    with FakeTensorMode():
        value = torch.empty(2, 30, 4, 8)
        shapes = torch.empty(2, 2, dtype=torch.int64)
        starts = torch.empty(2, dtype=torch.int64)
        loc = torch.empty(2, 7, 4, 2, 3, 2)
        attn = torch.empty(2, 7, 4, 2, 3)
        out = torch.ops.msda_amd.forward(value, shapes, starts, loc, attn, False, False)
        assert out.shape == (2, 7, 32)
        g = torch.empty(2, 7, 32)
        gv, gl, ga = torch.ops.msda_amd.backward(value, shapes, starts, loc, attn, g, True, True)
        assert gv.shape == value.shape and gl.shape == loc.shape and ga.shape == attn.shape
        ref = torch.empty(2, 7, 2, 2)
        out, lse = torch.ops.msda_amd.fused_forward(value, shapes, starts, ref, loc, attn, False, 1,
                                                    False)
        assert out.shape == (2, 7, 32) and lse.shape == (2, 7, 4) and lse.dtype == torch.float32
        grads = torch.ops.msda_amd.fused_backward(value, shapes, starts, ref, loc, attn, lse, out,
                                                  g, False, 1, True)
        assert [t.shape for t in grads] == [value.shape, ref.shape, loc.shape, attn.shape]


def test_backward_plan(lib, overrides):
    """Which grad_value path each preset's shapes take (host-only query)."""
    owner, dedup, direct, binned = 2, 1, 0, 3
    # decoder (B4 Q300 L4 K4, bf16): Q*K = 1200 per level, 64-byte rows
    assert lib.msda_backward_plan(4, 22223, 8, 32, 300, 4, 4, 2, 0) == owner
    assert lib.msda_backward_plan(4, 22223, 8, 32, 300, 4, 4, 2, 1) == owner  # deterministic
    assert lib.msda_backward_plan(2, 22223, 8, 32, 22223, 4, 4, 1, 1) == binned  # deterministic
    # encoder / Mask2Former: Q = S, far more samples per (b, m, level)
    assert lib.msda_backward_plan(2, 22223, 8, 32, 22223, 4, 4, 1, 0) == binned
    assert lib.msda_backward_plan(2, 21504, 8, 32, 21504, 3, 4, 0, 0) == binned
    assert lib.msda_backward_plan(2, 21504, 8, 32, 21504, 3, 4, 2, 0) == binned
    # binned path limits: head rows of 32, 64 or 128 bytes, D a power of two,
    # bookkeeping within grad_attention_weights, <= 1024 (b, m, level) groups
    assert lib.msda_backward_plan(2, 21504, 8, 64, 21504, 3, 4, 1, 0) == binned  # 128 B
    assert lib.msda_backward_plan(2, 21504, 8, 64, 21504, 3, 4, 0, 0) != binned  # 256 B
    assert lib.msda_backward_plan(2, 21504, 8, 24, 21504, 3, 4, 1, 0) == dedup   # D = 24
    assert lib.msda_backward_plan(2, 21504, 8, 8, 21504, 3, 4, 1, 0) != binned   # 16 B
    assert lib.msda_backward_plan(32, 21504, 8, 32, 21504, 4, 4, 1, 0) == binned  # 1024 groups
    # 33 batch elements: slices of at most 1024 groups (32 + 1) stay binned
    assert lib.msda_backward_plan(33, 21504, 8, 32, 21504, 4, 4, 1, 0) == binned
    assert lib.msda_backward_plan(1, 21504, 1025, 32, 21504, 1, 4, 1, 0) == dedup
    assert lib.msda_backward_plan(1, 600, 2, 32, 1100, 2, 2, 1, 0) == binned  # 2200 B / group
    assert lib.msda_backward_plan(1, 200000, 2, 32, 1100, 2, 2, 1, 0) == dedup  # bands > room
    # limits of the owner path: Q*K <= 2048, Q*D*elem <= 40960, rows of 16..256 bytes
    assert lib.msda_backward_plan(1, 600, 2, 32, 128, 2, 16, 1, 0) == owner  # Q*K = 2048
    assert lib.msda_backward_plan(1, 600, 2, 32, 128, 2, 17, 1, 0) != owner
    assert lib.msda_backward_plan(1, 600, 2, 32, 305, 2, 4, 1, 0) == owner   # 19520 B: 40 KB build
    assert lib.msda_backward_plan(1, 600, 2, 32, 640, 2, 2, 1, 0) == owner   # 40960 B
    assert lib.msda_backward_plan(1, 600, 2, 32, 641, 2, 2, 1, 0) != owner
    assert lib.msda_backward_plan(1, 600, 2, 32, 320, 2, 4, 0, 0) == owner   # 40960 B
    assert lib.msda_backward_plan(1, 600, 2, 32, 321, 2, 4, 0, 0) != owner
    assert lib.msda_backward_plan(1, 600, 2, 3, 100, 2, 4, 1, 0) == direct   # odd half row
    assert lib.msda_backward_plan(1, 600, 2, 128, 40, 2, 4, 1, 0) == owner   # 256-byte rows
    assert lib.msda_backward_plan(1, 600, 2, 256, 40, 2, 4, 1, 0) != owner
    # launch overrides
    overrides(BWD_OWNER=0)
    # decoder: the bookkeeping (2404 B per group) exceeds grad_attention_weights (2400 B)
    assert lib.msda_backward_plan(4, 22223, 8, 32, 300, 4, 4, 2, 0) == dedup
    assert lib.msda_backward_plan(4, 5600, 8, 32, 300, 4, 4, 2, 0) == binned
    overrides(BWD_BIN=0)
    assert lib.msda_backward_plan(4, 5600, 8, 32, 300, 4, 4, 2, 0) == dedup
    assert lib.msda_backward_plan(2, 22223, 8, 32, 22223, 4, 4, 1, 0) == dedup
    overrides(BWD_PRIV=0)
    assert lib.msda_backward_plan(4, 22223, 8, 32, 300, 4, 4, 2, 0) == direct
    # errors come back negated
    assert lib.msda_backward_plan(1, 1, 1, 1, 1, 1, 1, 9, 0) == -2
    assert lib.msda_backward_plan(-1, 1, 1, 1, 1, 1, 1, 0, 0) == -1


def test_deterministic_workspace_size(lib):
    # int64 accumulator (8 bytes per grad_value element) + the scale words;
    # none where the owner path (reproducible by construction) applies.
    assert lib.msda_deterministic_workspace_bytes(2, 22223, 8, 32, 22223, 4, 4, 1) == \
        2 * 22223 * 8 * 32 * 8 + 64
    assert lib.msda_deterministic_workspace_bytes(4, 22223, 8, 32, 300, 4, 4, 2) == 0
    assert lib.msda_deterministic_workspace_bytes(-1, 1, 1, 1, 1, 1, 1, 0) == -1
    assert lib.msda_deterministic_workspace_bytes(1, 1, 1, 1, 1, 1, 1, 9) == -1


def test_deterministic_flag_follows_torch():
    from msda_triton_amd.ops import _use_deterministic

    assert _use_deterministic(True) and not _use_deterministic(False)
    prev = torch.are_deterministic_algorithms_enabled()
    try:
        torch.use_deterministic_algorithms(True)
        assert _use_deterministic(None)
        torch.use_deterministic_algorithms(False)
        assert not _use_deterministic(None)
    finally:
        torch.use_deterministic_algorithms(prev)


def test_mmcv_shim_signature_and_validation():
    import inspect

    from msda_triton_amd import MSDeformAttnFunction, MultiScaleDeformableAttnFunction

    assert MSDeformAttnFunction is MultiScaleDeformableAttnFunction
    params = list(inspect.signature(MultiScaleDeformableAttnFunction.apply).parameters)
    assert params == ["value", "value_spatial_shapes", "value_level_start_index",
                      "sampling_locations", "attention_weights", "im2col_step"]
    value, shapes, starts, loc, attn = _inputs()
    with pytest.raises(ValueError, match="CUDA"):
        MultiScaleDeformableAttnFunction.apply(value, shapes, starts, loc, attn, 64)


# --- Projection entry points: argument checks before any launch ----------

def call_proj_fwd(lib, **kw):
    a = dict(x=16, w=16, b=None, w2=None, b2=None, m=None, y=16, y2=None, rows=4, cin=256, out=256,
             split=256, dtype=2)
    a.update(kw)
    return lib.msda_projection_forward(a["x"], a["w"], a["b"], a["w2"], a["b2"], a["m"], a["y"],
                                       a["y2"], a["rows"], a["cin"], a["out"], a["split"],
                                       a["dtype"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(dtype=5), 2),
    (dict(rows=-1), 1),
    (dict(split=300), 1),            # split > out_features
    (dict(split=0), 1),
    (dict(cin=20), 3),               # 40-byte bf16 rows: not a multiple of 16 bytes
    (dict(cin=520), 3),              # half-precision reduction longer than 512
    (dict(split=128), 1),            # two outputs but no weight2 / output2
    (dict(x=None), 1),
    (dict(x=8), 3),                  # input pointer not 16-byte aligned
    (dict(rows=0), 0),               # nothing to launch
])
def test_projection_forward_argument_errors(lib, kw, code):
    assert call_proj_fwd(lib, **kw) == code


def test_projection_backward_argument_errors(lib):
    def bwd(**kw):
        a = dict(x=16, w=16, w2=None, m=None, gy=16, gy2=None, gx=16, gw=None, gb=None, gw2=None,
                 gb2=None, ws=16, rows=4, cin=256, out=256, split=256, dtype=2)
        a.update(kw)
        return lib.msda_projection_backward(a["x"], a["w"], a["w2"], a["m"], a["gy"], a["gy2"],
                                            a["gx"], a["gw"], a["gb"], a["gw2"], a["gb2"], a["ws"],
                                            a["rows"], a["cin"], a["out"], a["split"], a["dtype"],
                                            None)
    assert bwd(split=100) == 3        # split not a multiple of 8 bf16 elements
    assert bwd(ws=None) == 1          # grad_input needs the workspace (transposed weight)
    assert bwd(gy=None) == 1
    assert bwd(out=600) == 3          # half grad_input reduction over 600 outputs
    assert bwd(gy=24) == 3            # misaligned grad_output
    assert bwd(rows=0, gx=None) == 0  # nothing requested, nothing launched
    assert lib.msda_projection_workspace_bytes(100, 20, 256, 2) == -1
    assert lib.msda_projection_workspace_bytes(100, 256, 256, 9) == -1


def test_projection_workspace_fits_the_noalloc_scratch():
    """msda_projection_backward_noalloc's scratch (64 MiB) holds the workspace
    (transposed weight + per-chunk weight-gradient partials) of every
    half-precision projection the library takes -- reductions of at most 512
    -- and of fp32 ones up to 512 x 512, at any row count (the chunk count is
    bounded by the CU count: 256 on MI355X, also the host-side default)."""
    lib = _native.load()
    limit = 64 << 20
    for dtype, feats in ((1, (16, 64, 128, 256, 384, 512)), (2, (16, 64, 128, 256, 384, 512)),
                         (0, (16, 64, 256, 512))):
        for cin in feats:
            for out in feats:
                for rows in (1, 1200, 88892, 10 ** 6, 10 ** 7):
                    need = lib.msda_projection_workspace_bytes(rows, cin, out, dtype)
                    assert 0 < need <= limit, (rows, cin, out, dtype, need)


def test_projection_rejects_cpu_tensors():
    from msda_triton_amd.projection import projection

    x = torch.randn(3, 16)
    w = torch.randn(8, 16)
    with pytest.raises(ValueError, match="CUDA"):
        projection(x, w)
