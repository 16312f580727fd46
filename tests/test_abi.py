"""C-ABI checks that need no GPU: the library loads, exports every entry point
declared in include/eimoe.h, and rejects bad arguments on the host before any
launch (error codes + messages), mirroring the reference's argument checks
(e.g. blocks/moe/base.py:145-146, modules/moe/base.py:67-68)."""
import ctypes
import re
from pathlib import Path

import pytest

from easyinfra_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "eimoe.h"


def header_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(eimoe_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_abi_version():
    lib = _lib.lib()
    assert lib.eimoe_abi_version() == 1


def test_every_header_function_is_exported_and_bound():
    names = header_functions()
    assert len(names) >= 12
    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    for n in names:
        assert hasattr(raw, n), f"{n} declared in eimoe.h but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def _rc(name, *args):
    return getattr(_lib.lib(), name)(*args)


def test_router_validation():
    assert _rc("eimoe_router_topk", None, 4, 8, 9, 1, None, None, None) == _lib.ERR_SHAPE
    assert "k=9" in _lib.last_error()
    assert _rc("eimoe_router_topk", None, 4, 600, 2, 1, None, None, None) == _lib.ERR_SHAPE
    assert _rc("eimoe_router_topk", None, 4, 8, 2, 1, None, None, None) == _lib.ERR_NULL
    assert "logits" in _lib.last_error()
    assert _rc("eimoe_router_topk", None, 0, 8, 2, 1, None, None, None) == _lib.EIMOE_OK  # empty batch
    assert _rc("eimoe_router_topk", None, -1, 8, 2, 1, None, None, None) == _lib.ERR_SHAPE


def test_align_validation():
    assert _rc("eimoe_align", None, 4, 2, 0, 0, None, None, None, None, None, None, 0, None) == _lib.ERR_SHAPE
    assert _rc("eimoe_align", None, 4, 2, -1, 8, None, None, None, None, None, None, 0, None) == _lib.ERR_SHAPE
    assert _rc("eimoe_align", None, 4, 40, 0, 8, None, None, None, None, None, None, 0, None) == _lib.ERR_SHAPE
    assert _rc("eimoe_align", None, 4, 2, 0, 8, None, None, None, None, None, None, 0, None) == _lib.ERR_NULL
    # the many-workgroup sort's chunk counts: none below 4096 routed pairs, one row of n_local per ~1024 pairs
    ws = _lib.lib().eimoe_align_workspace_bytes
    assert ws(1000, 4, 64) == 0
    assert ws(8192, 2, 8) == 16 * 8 * 4
    assert ws(16384, 8, 512) == 32 * 512 * 4                  # at most 16384 matrix cells


def test_route_align_validation():
    n = [None] * 7
    assert _rc("eimoe_route_align", None, 4, 8, 2, 1, 0, 0, *n, None) == _lib.ERR_SHAPE      # n_local 0
    assert _rc("eimoe_route_align", None, 4, 8, 9, 1, 0, 8, *n, None) == _lib.ERR_SHAPE      # k > E
    assert _rc("eimoe_route_align", None, 4, 8, 2, 1, -1, 8, *n, None) == _lib.ERR_SHAPE     # e_lo < 0
    assert _rc("eimoe_route_align", None, 4, 0, 1, 1, 0, 8, *n, None) == _lib.ERR_SHAPE      # E 0
    assert _rc("eimoe_route_align", None, 4, 8, 2, 1, 0, 8, *n, None) == _lib.ERR_NULL


def test_router_grouped_validation():
    f = "eimoe_router_grouped_topk"
    assert _rc(f, None, 4, 256, 8, 7, 4, None, 1, 1.0, None, None, None) == _lib.ERR_SHAPE    # 7 does not divide 256
    assert _rc(f, None, 4, 8, 2, 8, 4, None, 1, 1.0, None, None, None) == _lib.ERR_SHAPE      # groups of 1 expert
    assert _rc(f, None, 4, 256, 8, 8, 9, None, 1, 1.0, None, None, None) == _lib.ERR_SHAPE    # topk_group > n_group
    assert _rc(f, None, 4, 256, 33, 8, 4, None, 1, 1.0, None, None, None) == _lib.ERR_SHAPE   # k > 32
    assert _rc(f, None, 4, 1024, 8, 8, 4, None, 1, 1.0, None, None, None) == _lib.ERR_SHAPE   # E > 512
    assert _rc(f, None, 4, 256, 8, 8, 4, None, 1, 1.0, None, None, None) == _lib.ERR_NULL
    assert _rc(f, None, 0, 256, 8, 8, 4, None, 1, 1.0, None, None, None) == _lib.EIMOE_OK


def test_eplb_map_validation():
    f = "eimoe_eplb_map"
    assert _rc(f, None, 4, 0, None, 8, 2, None, None, None) == _lib.ERR_SHAPE    # k = 0
    assert _rc(f, None, 4, 2, None, 0, 2, None, None, None) == _lib.ERR_SHAPE    # no logical experts
    assert _rc(f, None, 4, 2, None, 8, 2, None, None, None) == _lib.ERR_NULL
    assert _rc(f, None, 0, 2, None, 8, 2, None, None, None) == _lib.EIMOE_OK


def test_moe_prologue_validation():
    f = "eimoe_moe_prologue"
    n = [None] * 3
    assert _rc(f, None, None, None, 1e-6, None, 4, 100, 8, 0, *n, None, 0, None) == _lib.ERR_ALIGN    # H % 64
    assert _rc(f, None, None, None, 1e-6, None, 4, 16384, 8, 0, *n, None, 0, None) == _lib.ERR_ALIGN  # H > 8192
    assert _rc(f, None, None, None, 1e-6, None, 4, 4096, 48, 0, *n, None, 0, None) == _lib.ERR_SHAPE  # 48 experts
    assert _rc(f, None, None, None, 1e-6, None, 4, 4096, 8, 0, *n, None, 0, None) == _lib.ERR_NULL
    assert _rc(f, None, None, None, 1e-6, None, 0, 4096, 8, 0, *n, None, 0, None) == _lib.EIMOE_OK
    # the router GEMM's workspace: offsets, then K-split planes while the tiles do not fill the chip
    ws = _lib.lib().eimoe_moe_prologue_workspace_bytes
    assert ws(8192, 4096, 8) == 0                                    # dotted in the same pass
    assert ws(4096, 7168, 256) == 256 + 8 * 4096 * 256 * 4           # 64 tiles of 128 x 128: 8 planes
    assert ws(16384, 2048, 128) == 256 + 4 * 16384 * 128 * 4         # 128 tiles: 4 planes of 512
    assert ws(4100, 1024, 192) == 256                                # 771 tiles of 16 x 64: no split
    assert _rc(f, 1, 1, 1, 1e-6, 1, 4096, 7168, 256, 0, 1, 2, 3, 4, 256, None) == _lib.ERR_WORKSPACE
    assert _rc(f, 1, 1, 1, 1e-6, 1, 262144, 4096, 256, 0, 1, 2, 3, 4, 1 << 40, None) == _lib.ERR_SHAPE  # normed 2 GiB


def test_gemm_validation():
    # H not a multiple of 64
    assert _rc("eimoe_gemm_gate_up_silu", 1, None, 4, 100, 1, _lib.BF16, None, 100, 64, 1, 1, 1, 4, 1, 0,
               None) == _lib.ERR_ALIGN
    # I not a multiple of 32
    assert _rc("eimoe_gemm_gate_up_silu", 1, None, 4, 128, 1, _lib.BF16, None, 128, 40, 1, 1, 1, 4, 1, 0,
               None) == _lib.ERR_ALIGN
    # fp8 weights need scales
    assert _rc("eimoe_gemm_gate_up_silu", 1, None, 4, 128, 1, _lib.FP8, None, 128, 64, 1, 1, 1, 4, 1, 0,
               None) == _lib.ERR_NULL
    # bad dtype / segment count / tile
    assert _rc("eimoe_gemm_gate_up_silu", 1, None, 4, 128, 1, 7, None, 128, 64, 1, 1, 1, 4, 1, 0,
               None) == _lib.ERR_DTYPE
    assert _rc("eimoe_gemm_gate_up_silu", 1, None, 4, 128, 1, _lib.BF16, None, 128, 64, 1, 2000, 1, 4, 1, 0,
               None) == _lib.ERR_SHAPE
    assert _rc("eimoe_gemm_gate_up_silu", 1, None, 4, 128, 1, _lib.BF16, None, 128, 64, 1, 1, 1, 4, 1, 9,
               None) == _lib.ERR_SHAPE
    assert _rc("eimoe_gemm_gate_up_silu", 1, None, 4, 128, 1, _lib.BF16, None, 128, 64, 1, 1, 1, 4, 1,
               _lib.TILE_64x128 + 1, None) == _lib.ERR_SHAPE
    # the 64x128 tile writes 64 gate/up output columns: I = 96 does not fit it
    assert _rc("eimoe_gemm_gate_up_silu", 1, None, 4, 128, 1, _lib.BF16, None, 128, 96, 1, 1, 1, 4, 1,
               _lib.TILE_64x128, None) == _lib.ERR_ALIGN
    # tile whose output width does not divide I
    assert _rc("eimoe_gemm_gate_up_silu", 1, None, 4, 128, 1, _lib.BF16, None, 128, 96, 1, 1, 1, 4, 1,
               _lib.TILE_256x256, None) == _lib.ERR_ALIGN
    # down: I must be a multiple of 64*k_split
    assert _rc("eimoe_gemm_down", 1, 192, 1, _lib.BF16, None, 128, 1, 1, 1, 4, 1, _lib.F32, 2, 0,
               None) == _lib.ERR_ALIGN
    assert _rc("eimoe_gemm_down", 1, 192, 1, _lib.BF16, None, 128, 1, 1, 1, 4, 1, 5, 1, 0, None) == _lib.ERR_DTYPE
    # zero rows is a no-op
    assert _rc("eimoe_gemm_down", None, 192, None, _lib.BF16, None, 128, None, 1, 1, 0, None, _lib.F32, 1, 0,
               None) == _lib.EIMOE_OK


def test_combine_and_quant_validation():
    assert _rc("eimoe_combine", 1, _lib.F32, 1, 0, 1, 1, 4, 2, 100, None, 0, 1, _lib.F32, None) == _lib.ERR_ALIGN
    assert _rc("eimoe_combine", 1, 3, 1, 0, 1, 1, 4, 2, 128, None, 0, 1, _lib.F32, None) == _lib.ERR_DTYPE
    assert _rc("eimoe_combine", None, _lib.F32, 1, 0, 1, 1, 4, 2, 128, None, 0, 1, _lib.F32, None) == _lib.ERR_NULL
    assert _rc("eimoe_quantize_rows_fp8", None, _lib.FP8, 4, 4, None, None, None) == _lib.ERR_DTYPE
    assert _rc("eimoe_quantize_rows_fp8", None, _lib.F32, 0, 4, None, None, None) == _lib.EIMOE_OK


def test_fused_validation_and_workspace():
    f = "eimoe_fused_moe"
    base = dict(x=1, logits=1, T=16, H=256, I=128, E=8, k=2, wgu=1, wd=1, wdt=_lib.BF16, sgu=None, sd=None, e_lo=0,
                n_local=8, shgu=None, shd=None, Is=0, flags=1, out=1, odt=_lib.BF16, ws=1, wsb=1 << 30, ids=None,
                w=None, stream=None)

    def call(**kw):
        a = dict(base, **kw)
        return _rc(f, *a.values())

    assert call(k=9) == _lib.ERR_SHAPE
    assert call(e_lo=4, n_local=8) == _lib.ERR_SHAPE            # window outside [0,E)
    assert call(H=100) == _lib.ERR_ALIGN
    assert call(I=96) == _lib.ERR_ALIGN
    assert call(wdt=_lib.FP8) == _lib.ERR_NULL                   # fp8 without scales
    assert call(Is=256) == _lib.ERR_NULL                         # shared size without weights
    assert call(wsb=16) == _lib.ERR_WORKSPACE
    assert "workspace" in _lib.last_error()
    # extents past the GEMMs' 32-bit buffer offsets are refused before any launch
    assert call(T=131072, H=8192, I=128) == _lib.ERR_SHAPE        # x: 2 GiB
    assert "x (" in _lib.last_error()
    assert call(T=65536, H=256, I=8192, k=2) == _lib.ERR_SHAPE     # h: T*k x I = 2 GiB
    assert call(H=8192, I=65536, T=16) == _lib.ERR_SHAPE           # one expert's gate/up weights
    assert call(T=0) == _lib.EIMOE_OK
    ws = _lib.lib().eimoe_fused_moe_workspace_bytes(16, 256, 128, 8, 2, 8, 0, _lib.BF16, 1)
    ws_sh = _lib.lib().eimoe_fused_moe_workspace_bytes(16, 256, 128, 8, 2, 8, 256, _lib.BF16, 1)
    ws_f32 = _lib.lib().eimoe_fused_moe_workspace_bytes(16, 256, 128, 8, 2, 8, 0, _lib.F32, 1)
    # the per-assignment outputs y are fp32 whatever the output type
    assert 0 < ws < ws_sh and ws == ws_f32
    # h (A*I bf16) and y (A*H fp32) dominate: at least that much
    assert ws >= 32 * 128 * 2 + 32 * 256 * 4


def test_fused_down_split_query():
    """eimoe_fused_moe_down_split: the layer's own choice (a power of two dividing the K steps), 0
    where the workspace query refuses the arguments."""
    L = _lib.lib()
    for T, H, I, E, k, n in [(8192, 4096, 14336, 8, 2, 8), (64, 4096, 14336, 8, 2, 8), (2048, 2048, 768, 128, 8, 32),
                             (4096, 2048, 1408, 64, 6, 64), (1, 256, 128, 8, 2, 8)]:
        ks = L.eimoe_fused_moe_down_split(T, H, I, E, k, n, 0, _lib.BF16, 1)
        assert ks in (1, 2, 4, 8) and I % (64 * ks) == 0
    assert L.eimoe_fused_moe_down_split(16, 256, 128, 8, 0, 8, 0, _lib.BF16, 1) == 0


def test_static_scratch_limit_matches_the_documented_token_count():
    """The largest Mixtral-8x7B layer (H 4096, I 14336, 8 experts, top-2) the 64 MiB static scratch
    holds, as the header states it: 545 tokens with bf16 or fp32 output."""
    L = _lib.lib()
    cap = L.eimoe_fused_moe_static_bytes()
    assert cap == 64 << 20
    for odt in (_lib.BF16, _lib.F32):
        need = lambda T: L.eimoe_fused_moe_workspace_bytes(T, 4096, 14336, 8, 2, 8, 0, odt, 1)
        assert need(545) <= cap < need(546)


def test_ops_refuse_cpu_tensors():
    torch = pytest.importorskip("torch")
    from easyinfra_amd import ops
    with pytest.raises(ValueError):
        ops.router_topk(torch.zeros(4, 8), 2)


def test_bench_refuses_more_than_one_gpu():
    # one GPU per box: the multi-GPU launch exits with a message instead of measuring
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout.strip() == ""
