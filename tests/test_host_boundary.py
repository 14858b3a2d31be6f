"""CPU checks of the C-ABI boundary and the host logic (no GPU compute)."""
import ctypes
import os
import re
import subprocess
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pack3d_hip.h")


PROBE_HEADER = os.path.join(ROOT, "include", "pack3d_probe.h")


def _declared(header=HEADER):
    text = open(header).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(p3d_\w+)\s*\(", text, re.M)))


def test_probe_library_is_separate_from_the_product():
    """The issue-rate probe is measurement scaffolding: its own library
    exports what include/pack3d_probe.h declares, and the product library
    does not export it."""
    from pack3d_amd import _lib
    probe = ctypes.CDLL(_lib.PROBE_PATH)
    for name in _declared(PROBE_HEADER):
        assert hasattr(probe, name), name
    product = ctypes.CDLL(_lib.LIB_PATH)
    assert not hasattr(product, "p3d_probe_issue_rates")
    assert "p3d_probe_issue_rates" not in _declared()


def test_library_exports_every_declared_symbol():
    from pack3d_amd import _lib
    names = _declared()
    assert len(names) >= 14
    handle = ctypes.CDLL(_lib.LIB_PATH)
    for name in names:
        assert hasattr(handle, name), name
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures must cover exactly the header"


def test_struct_mirrors_match_c_sizes():
    from pack3d_amd import _lib
    out = (ctypes.c_int64 * 6)()
    assert _lib.lib().p3d_struct_sizes(out) == 0
    assert list(out) == [ctypes.sizeof(_lib.View), ctypes.sizeof(_lib.Rope), ctypes.sizeof(_lib.PoolArgs),
                         ctypes.sizeof(_lib.AttnArgs), ctypes.sizeof(_lib.BwdArgs),
                         ctypes.sizeof(_lib.ProjectArgs)]
    header = open(os.path.join(ROOT, "include", "pack3d_hip.h")).read()
    version = int(re.search(r"#define P3D_ABI_VERSION (\d+)", header).group(1))
    assert _lib.lib().p3d_abi_version() == version == _lib.ABI_VERSION


def test_entry_points_reject_bad_arguments_before_launch():
    from pack3d_amd import _lib
    grid = _lib.i64x3((4, 4, 4))
    bad_block = _lib.i64x3((3, 4, 4))
    rad = _lib.i64x3((1, 1, 1))
    rc = _lib.lib().p3d_build_layout(grid, bad_block, rad, 0, None, None, None, None, None, None)
    assert rc == 1 and b"divisible" in _lib.lib().p3d_last_error()
    with pytest.raises(RuntimeError, match="null args"):
        _lib.call("p3d_pool_fwd", None, None)
    args = _lib.AttnArgs()
    with pytest.raises(RuntimeError, match="dtype|counts"):
        args.dtype = 7
        _lib.call("p3d_attn_fwd_grid", args, None)
    # Weight gradient: widths the kernel does not take (never dereferenced).
    bf16 = _lib.DTYPES[torch.bfloat16]
    for out_f, in_f, msg in ((12, 192, "out_features"), (8, 48, "in_features"), (8, 288, "in_features"),
                             (8, 2304, "in_features")):
        with pytest.raises(RuntimeError, match=msg):
            _lib.call("p3d_weight_grad", 16, out_f, 16, in_f, 16, 16, 100, out_f, in_f, 1, bf16, None)
    with pytest.raises(RuntimeError, match="null pointer"):
        _lib.call("p3d_weight_grad", None, 8, 16, 32, 16, 16, 100, 8, 32, 1, bf16, None)
    # Transposed copies: 16-bit types and token counts a multiple of 8 only.
    src = _lib.View(16, 0, 0, 64)
    for n, d, dt, msg in ((12, 64, bf16, "multiple of 8"), (16, 64, _lib.P3D_F32, "fp16 or bf16"),
                          (16, 12, bf16, "head_dim")):
        with pytest.raises(RuntimeError, match=msg):
            _lib.call("p3d_transpose_rows", src, 16, 1, 1, n, d, dt, None)


def test_import_without_gpu_and_no_oracle_import():
    code = ("import sys, pack3d_amd; assert 'oracle' not in sys.modules; "
            "assert not any(m.startswith('oracle') for m in sys.modules)")
    subprocess.run([sys.executable, "-c", code], check=True, cwd=ROOT)


def test_product_sources_never_reference_the_oracle():
    pkg = os.path.join(ROOT, "pack3d_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".cpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text, f


@pytest.mark.parametrize("kwargs", [{"grid_shape": (3, 4, 4)}, {"radius": -1}, {"block_shape": (0, 2, 2)},
                                    {"layout": "unknown"}, {"pool_size": True}, {"radius": 3},
                                    {"block_shape": (8, 8, 8), "grid_shape": (8, 8, 8)}])
def test_build_layout_rejects_before_launch(kwargs):
    from pack3d_amd import build_layout
    args = {"grid_shape": (4, 4, 4), **kwargs}
    with pytest.raises(ValueError):
        build_layout(**args)


def test_prepare_geometry_shape_checks():
    from pack3d_amd import prepare_geometry
    with pytest.raises(ValueError, match="rank-two"):
        prepare_geometry(torch.zeros(3, dtype=torch.int32), torch.zeros(1, 3, dtype=torch.int32), 1)
    with pytest.raises(ValueError, match="nonempty"):
        prepare_geometry(torch.zeros(0, 2, dtype=torch.int32), torch.zeros(1, 3, dtype=torch.int32), 1)
    with pytest.raises(ValueError, match="pool_size"):
        prepare_geometry(torch.zeros(3, 1, dtype=torch.int32), torch.zeros(1, 3, dtype=torch.int32), 0)
    with pytest.raises(ValueError, match="at most 128"):
        prepare_geometry(torch.zeros(3, 129, dtype=torch.int32), torch.zeros(1, 3, dtype=torch.int32), 1)


@pytest.mark.parametrize("kwargs", [{"heads": 3}, {"temperature": 0}, {"backend": "auto"},
                                    {"backend": "reference"}, {"position_encoding": "none"},
                                    {"head_dim": 40}])
def test_layer_rejects_unsupported(kwargs):
    from pack3d_amd import PACK3DAttention
    with pytest.raises(ValueError):
        PACK3DAttention(32, **kwargs)


def test_layer_parameters_match_reference_names_and_init_stream():
    from oracle.pack3d_oracle import PACK3DAttention as Oracle
    from pack3d_amd import PACK3DAttention
    torch.manual_seed(5)
    a = PACK3DAttention(192, heads=4, kv_heads=4, head_dim=48, block_volume=64)
    torch.manual_seed(5)
    b = Oracle(192, heads=4, kv_heads=4, head_dim=48, block_volume=64)
    sa, sb = a.state_dict(), b.state_dict()
    assert list(sa) == list(sb)
    for k in sa:
        assert torch.equal(sa[k], sb[k]), k


def test_core_requires_hip_device_no_fallback():
    from oracle.pack3d_oracle import prepare_geometry as oracle_prepare
    from pack3d_amd import pack3d_hip
    from pack3d_amd.geometry import Pack3DGeometry, _SEAL
    from tests._cases import make_case
    inputs, nb, blocks, pool = make_case(d=48)
    og = oracle_prepare(nb, blocks, pool)
    geom = Pack3DGeometry(og.neighbors, og.reverse_neighbors, og.blocks, pool, og.num_tokens, _SEAL)
    with pytest.raises(ValueError, match="hip backend requires"):
        pack3d_hip(*inputs, geom)
    inputs[0] = inputs[0][..., :40]
    with pytest.raises(ValueError):
        pack3d_hip(*inputs, geom)


def test_param_f32_cache_follows_updates():
    import torch
    from pack3d_amd.core import param_f32
    p = torch.nn.Parameter(torch.arange(6, dtype=torch.bfloat16))
    a = param_f32(p)
    assert a.dtype == torch.float32 and torch.equal(a, p.detach().float())
    assert param_f32(p) is a  # unchanged parameter: the cached copy
    with torch.no_grad():
        p.add_(1)
    b = param_f32(p)
    assert b is not a and torch.equal(b, p.detach().float())  # in-place update: a fresh copy
    q = torch.arange(4, dtype=torch.float32)
    assert param_f32(q).data_ptr() == q.data_ptr()  # fp32 contiguous: no copy


def test_grid_tag_reads_the_reference_radius_one_tag():
    """A geometry shaped like the reference's (no ``_grid``): its radius-one tag
    (geometry.py:18-19,262-265) selects the brick kernels; other radii carry no
    tag until adopt_layout proves one."""
    import oracle.pack3d_oracle as ref
    from pack3d_amd.geometry import _stencil_radii, grid_tag
    from tests._refobjects import reference_layout
    lay = reference_layout(ref.build_layout((4, 16, 64), (2, 2, 2), radius=1, pool_size=2))
    tag = grid_tag(lay.geometry)
    assert tag[0] == (4, 16, 64) and tag[1] == (1, 1, 1)
    assert tag[2].dtype == torch.int32 and torch.equal(tag[2], lay.order.argsort().to(torch.int32))
    raster = reference_layout(ref.build_layout((4, 16, 64), (2, 2, 2), radius=1, layout="raster_block"))
    assert grid_tag(raster.geometry) == ((4, 16, 64), (1, 1, 1), None)
    assert grid_tag(reference_layout(ref.build_layout((8, 8, 8), (4, 4, 4), radius=2)).geometry) is None
    assert grid_tag(reference_layout(ref.build_layout((2, 4, 4), (2, 2, 2), radius=1)).geometry) is None
    assert _stencil_radii(125) == [(2, 2, 2)]
    assert sorted(_stencil_radii(45)) == [(1, 1, 2), (1, 2, 1), (2, 1, 1)]


def test_core_rejects_geometry_tables_that_are_not_int32():
    import oracle.pack3d_oracle as ref
    from pack3d_amd import pack3d_hip
    from tests._cases import make_case
    from tests._refobjects import RefGeometry
    inputs, nb, blocks, pool = make_case()
    g = ref.prepare_geometry(nb, blocks, pool)
    wide = RefGeometry(g.neighbors.long(), g.reverse_neighbors, g.blocks, g.pool_size, g.num_tokens)
    with pytest.raises(ValueError, match="int32"):
        pack3d_hip(*inputs, wide)


def test_blocks_consecutive_recognises_build_layout_blocks():
    """The fused projection pooling takes geometries whose fine block f is
    rows 64 f .. 64 f + 63 in slot order; any other table (rows swapped,
    other slot counts, an in-place change after a first check) does not."""
    import types

    import oracle.pack3d_oracle as ref
    from pack3d_amd.geometry import blocks_consecutive
    from tests._refobjects import reference_layout

    def geom(blocks):
        g = types.SimpleNamespace(blocks=blocks, num_tokens=blocks.numel())
        g.tensors = (blocks,)
        return g

    lay = reference_layout(ref.build_layout((4, 8, 8), (4, 4, 4), radius=1, pool_size=1))
    assert blocks_consecutive(lay.geometry)
    blocks = torch.arange(4 * 64, dtype=torch.int32).view(4, 64)
    g = geom(blocks.clone())
    assert blocks_consecutive(g) and blocks_consecutive(g)
    g.blocks[0, :2] = g.blocks[0, :2].flip(0)      # in place: the cached answer is dropped
    assert not blocks_consecutive(g)
    swapped = blocks.clone()
    swapped[[1, 2]] = swapped[[2, 1]]
    assert not blocks_consecutive(geom(swapped))
    assert not blocks_consecutive(geom(torch.arange(4 * 8, dtype=torch.int32).view(4, 8)))


def test_project_pool_answers_unsupported_before_launch():
    """p3d_project_pool refuses shapes it does not take with P3D_EUNSUPPORTED
    and malformed arguments with P3D_EINVAL, before touching any pointer."""
    from pack3d_amd import _lib
    bf16 = _lib.DTYPES[torch.bfloat16]
    fake = 1 << 20   # 16-byte aligned, never dereferenced
    h, g, d, dim, n = 4, 4, 48, 192, 4096
    args = _lib.ProjectArgs(fake, fake, fake, fake, fake, fake, fake, fake, fake, fake, n, dim, h * d, 4 * g * d,
                            h, bf16, bf16, bf16, 1e-5)
    pool = _lib.PoolArgs()
    pool.batch, pool.kv_heads, pool.tokens, pool.head_dim, pool.dtype = 1, g, n, d, bf16
    pool.fine_blocks, pool.slots, pool.pool_size, pool.summaries = n // 64, 64, 1, n // 64
    pool.temperature, pool.key_scale = 1.0, 1.0
    pool.weight = pool.bias = pool.sk = pool.svt = pool.sk_norm_max = fake
    pool.rope.table = pool.rope.pairs = pool.rope.coords = fake
    lib = _lib.lib()
    for field, value in (("pool_size", 2), ("slots", 32)):
        setattr(pool, field, value)
        assert lib.p3d_project_pool(args, pool, 1, None) == _lib.P3D_EUNSUPPORTED
        setattr(pool, field, {"pool_size": 1, "slots": 64}[field])
    pool.kv_heads = 2       # kv_out no longer 4 * kv_heads * head_dim
    assert lib.p3d_project_pool(args, pool, 1, None) == 1
    assert b"kv_out" in lib.p3d_last_error()
    pool.kv_heads = g
    pool.dtype = _lib.DTYPES[torch.float16]
    assert lib.p3d_project_pool(args, pool, 1, None) == 1
    with pytest.raises(RuntimeError, match="null args"):
        _lib.call("p3d_project_pool", None, None, 0, None)
