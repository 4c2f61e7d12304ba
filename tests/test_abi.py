"""CPU tests of the C-ABI library: it loads, exports every symbol include/kmoe.h
declares, and its host-side argument validation rejects bad calls with the
documented status codes (no kernel is launched on these paths)."""
import ctypes

import pytest

from kmoe import _lib

NULL = None


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_exports_every_header_symbol(lib):
    names = _lib.header_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding covers the whole header
    assert sorted(_lib._SIGNATURES) == names


def test_version_and_sizes(lib):
    assert lib.kmoe_abi_version() == 2
    assert lib.kmoe_padded_ff(2816) == 2816 and lib.kmoe_padded_ff(352) == 384
    assert lib.kmoe_router_partials_len(16384, 16) == 256 * 17
    # 32-token router blocks when ceil(T/32) workgroups fit the 256 compute units at once
    assert lib.kmoe_router_block_tokens(16384) == 64 and lib.kmoe_router_block_tokens(8193) == 64
    assert lib.kmoe_router_block_tokens(8192) == 32 and lib.kmoe_router_block_tokens(1) == 32
    assert lib.kmoe_router_partials_len(8192, 16) == 256 * 17 and lib.kmoe_router_partials_len(33, 4) == 2 * 5
    # packed rows carry 128 bytes of padding after the K-contiguous data
    assert lib.kmoe_packed_w13_bytes(16, 2048, 2816, _lib.DTYPE_BF16) == 16 * 2 * 2816 * (2048 * 2 + 128)
    assert lib.kmoe_packed_w3_bytes(16, 2048, 2816, _lib.DTYPE_FP8_E4M3) == 16 * 2048 * (2816 + 128)
    assert lib.kmoe_dispatch_workspace_bytes(16384, 2, 16) >= 2 * 128 * 16 * 4


def _err(lib, name, *args):
    rc = getattr(lib, name)(*args)
    return rc, lib.kmoe_last_error().decode()


FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first


def test_router_validation(lib):
    rc, msg = _err(lib, "kmoe_router", NULL, NULL, 16, 64, FAKE, FAKE, 8, NULL, 2, FAKE, FAKE, FAKE, NULL, NULL)
    assert rc == -1 and "null" in msg
    rc, msg = _err(lib, "kmoe_router", FAKE, NULL, 16, 65, FAKE, FAKE, 8, NULL, 2, FAKE, FAKE, FAKE, NULL, NULL)
    assert rc == -2 and "d=65" in msg
    rc, msg = _err(lib, "kmoe_router", FAKE, NULL, 16, 64, FAKE, FAKE, 65, NULL, 2, FAKE, FAKE, FAKE, NULL, NULL)
    assert rc == -2 and "E=65" in msg
    rc, msg = _err(lib, "kmoe_router", FAKE, NULL, 16, 64, FAKE, FAKE, 8, NULL, 9, FAKE, FAKE, FAKE, NULL, NULL)
    assert rc == -2 and "k=9" in msg
    # at most 8 picks per token, however many experts
    rc, msg = _err(lib, "kmoe_router", FAKE, NULL, 16, 64, FAKE, FAKE, 64, NULL, 9, FAKE, FAKE, FAKE, NULL, NULL)
    assert rc == -2 and "k=9" in msg
    rc, _ = _err(lib, "kmoe_router", FAKE, NULL, 16, 64, FAKE, FAKE, 8, NULL, 2, FAKE, NULL, FAKE, NULL, NULL)
    assert rc == -1


def test_dispatch_validation(lib):
    args = [FAKE, NULL, 16, 64, FAKE, FAKE, _lib.DTYPE_F32, 2, 8, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
            _lib.DTYPE_BF16, NULL, FAKE, 1 << 20, NULL]
    bad = list(args)
    bad[6] = 7
    assert _err(lib, "kmoe_dispatch", *bad)[0] == -3
    bad = list(args)
    bad[16] = _lib.DTYPE_FP8_E4M3  # fp8 needs a scale buffer
    assert _err(lib, "kmoe_dispatch", *bad)[0] == -1
    bad = list(args)
    bad[19] = 8  # workspace too small
    rc, msg = _err(lib, "kmoe_dispatch", *bad)
    assert rc == -4 and "workspace" in msg
    bad = list(args)
    bad[7] = 9  # k > 8
    assert _err(lib, "kmoe_dispatch", *bad)[0] == -2


def test_gemm_and_combine_validation(lib):
    assert _err(lib, "kmoe_gemm_gate_up", FAKE, NULL, _lib.DTYPE_BF16, FAKE, 0, 64, 64, 16, FAKE, NULL, FAKE,
                NULL)[0] == -2
    assert _err(lib, "kmoe_gemm_gate_up", FAKE, NULL, _lib.DTYPE_F32, FAKE, 4, 64, 64, 16, FAKE, NULL, FAKE,
                NULL)[0] == -3
    assert _err(lib, "kmoe_gemm_down", FAKE, NULL, _lib.DTYPE_FP8_E4M3, FAKE, 4, 64, 64, 16, FAKE, NULL, FAKE,
                NULL)[0] == -1
    rc, msg = _err(lib, "kmoe_gemm_gate_up", FAKE, FAKE, _lib.DTYPE_FP8_E4M3, FAKE, 4, 64, 64, 16, FAKE, FAKE,
                   FAKE, NULL)
    assert rc == -2 and "128" in msg
    assert _err(lib, "kmoe_combine", FAKE, 64, FAKE, FAKE, 0, NULL, NULL, 4, FAKE, _lib.DTYPE_BF16, NULL)[0] == -2
    assert _err(lib, "kmoe_combine", FAKE, 64, FAKE, FAKE, 2, NULL, NULL, 4, FAKE, _lib.DTYPE_FP8_E4M3,
                NULL)[0] == -3
    assert _err(lib, "kmoe_pack_weights", FAKE, FAKE, FAKE, _lib.DTYPE_BF16, 4, 64, 64, _lib.DTYPE_FP8_E4M3,
                FAKE, NULL, FAKE, NULL, NULL)[0] == -1
    # the residual-dropout combine: residual and keep mask required, keep_scale = 1/(1-p) >= 1
    rc, msg = _err(lib, "kmoe_combine_residual_dropout", FAKE, 64, FAKE, FAKE, 2, NULL, NULL, FAKE, NULL, 1.25, 4,
                   FAKE, _lib.DTYPE_BF16, NULL)
    assert rc == -1 and "keep" in msg
    rc, msg = _err(lib, "kmoe_combine_residual_dropout", FAKE, 64, FAKE, FAKE, 2, NULL, NULL, FAKE, FAKE, 0.5, 4,
                   FAKE, _lib.DTYPE_BF16, NULL)
    assert rc == -2 and "keep_scale" in msg
    assert _err(lib, "kmoe_combine_residual_dropout", FAKE, 60, FAKE, FAKE, 2, NULL, NULL, FAKE, FAKE, 1.25, 4,
                FAKE, _lib.DTYPE_BF16, NULL)[0] == -2


def test_select_validation(lib):
    assert _err(lib, "kmoe_ec_select", FAKE, 1, 100, 4, 101, 1, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, NULL, 0,
                NULL)[0] == -2
    assert _err(lib, "kmoe_ec_select", FAKE, 1, 100000, 4, 10, 1, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, NULL, 0,
                NULL)[0] == -6
    # the transposed-logits workspace: B*S*E floats, checked before any launch
    assert lib.kmoe_ec_workspace_bytes(2, 100, 4) == 2 * 100 * 4 * 4
    assert _err(lib, "kmoe_ec_select", FAKE, 2, 100, 4, 10, 1, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                2 * 100 * 4 * 4 - 1, NULL)[0] == -4
    assert _err(lib, "kmoe_mod_select", FAKE, 2, 100, 64, FAKE, 0, FAKE, FAKE, FAKE, FAKE, FAKE, NULL, 0,
                NULL)[0] == -2
    assert _err(lib, "kmoe_aux_loss", NULL, 16, 4, NULL, 2, 0.01, 0.001, FAKE, NULL)[0] == -1
    assert _err(lib, "kmoe_balanced_topk", FAKE, 100, 4, 5, FAKE, FAKE, FAKE, 1024, NULL)[0] == -2  # k > E
    assert _err(lib, "kmoe_balanced_topk", FAKE, 100, 4, 2, FAKE, FAKE, FAKE, 4, NULL)[0] == -4  # workspace


def test_dispatch_noalloc_validation(lib):
    """The allocation-free dispatch rejects, before any GPU call, sizes whose histograms do
    not fit its fixed device scratch, and bad arguments like kmoe_dispatch."""
    args = [FAKE, NULL, 16, 64, FAKE, FAKE, _lib.DTYPE_F32, 2, 8, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
            _lib.DTYPE_BF16, NULL, NULL]
    big = list(args)
    big[2] = 1 << 21  # T = 2M tokens at E = 64: 16 MiB of histograms > 4 MiB
    big[8] = 64
    rc, msg = _err(lib, "kmoe_dispatch_noalloc", *big)
    assert rc == -4 and "scratch" in msg
    bad = list(args)
    bad[6] = 7
    assert _err(lib, "kmoe_dispatch_noalloc", *bad)[0] == -3
    bad = list(args)
    bad[0] = NULL
    assert _err(lib, "kmoe_dispatch_noalloc", *bad)[0] == -1
    # the largest size that fits is accepted by the size check (T*E = 2^25 - 8192 for k=2)
    assert lib.kmoe_dispatch_workspace_bytes((1 << 21) - 512, 2, 16) <= 4 << 20


def test_counted_dispatch_and_router_hist_validation(lib):
    args = [FAKE, NULL, 16, 64, FAKE, FAKE, _lib.DTYPE_F32, 2, 8, 0, NULL, FAKE, FAKE, FAKE, FAKE, FAKE, NULL,
            _lib.DTYPE_BF16, NULL, FAKE, 1 << 20, NULL]
    rc, msg = _err(lib, "kmoe_dispatch_counted", *args)
    assert rc == -1 and "block_counts" in msg
    good = list(args)
    good[10] = FAKE
    good[20] = 8  # workspace too small
    assert _err(lib, "kmoe_dispatch_counted", *good)[0] == -4
    rc, msg = _err(lib, "kmoe_router_hist", FAKE, NULL, 16, 64, FAKE, FAKE, 8, NULL, 2, FAKE, FAKE, FAKE, NULL, NULL,
                   NULL, NULL)
    assert rc == -1 and "block_counts" in msg


def test_counted_dispatch_aux_validation(lib):
    # kmoe_dispatch_counted's arguments, then partials, w_lb, w_z, aux_out, stream
    base = [FAKE, NULL, 16, 64, FAKE, FAKE, _lib.DTYPE_F32, 2, 8, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, NULL,
            _lib.DTYPE_BF16, NULL, FAKE, 1 << 20]
    rc, msg = _err(lib, "kmoe_dispatch_counted_aux", *base, NULL, 0.01, 0.001, FAKE, NULL)
    assert rc == -1 and "partials" in msg
    rc, msg = _err(lib, "kmoe_dispatch_counted_aux", *base, FAKE, 0.01, 0.001, NULL, NULL)
    assert rc == -1 and "aux_out" in msg
    no_t = list(base)
    no_t[2] = 0
    rc, msg = _err(lib, "kmoe_dispatch_counted_aux", *no_t, FAKE, 0.01, 0.001, FAKE, NULL)
    assert rc == -2 and "T must be > 0" in msg
    small = list(base)
    small[20] = 8
    assert _err(lib, "kmoe_dispatch_counted_aux", *small, FAKE, 0.01, 0.001, FAKE, NULL)[0] == -4


def test_norm_and_mod_backward_validation(lib):
    """Argument checks of the block / MoD training entry points (no launch on failure)."""
    BF, F32 = _lib.DTYPE_BF16, _lib.DTYPE_F32
    assert _err(lib, "kmoe_rmsnorm", FAKE, BF, NULL, F32, 1e-5, 16, 64, FAKE, FAKE, NULL, NULL, NULL)[0] == -1
    assert _err(lib, "kmoe_rmsnorm", FAKE, BF, FAKE, F32, 1e-5, 16, 64, FAKE, FAKE, FAKE, NULL, NULL)[0] == -1
    assert _err(lib, "kmoe_rmsnorm", FAKE, 7, FAKE, F32, 1e-5, 16, 64, FAKE, FAKE, NULL, NULL, NULL)[0] == -3
    assert _err(lib, "kmoe_rmsnorm", FAKE, BF, FAKE, F32, 1e-5, 16, 60, FAKE, FAKE, NULL, NULL, NULL)[0] == -2
    assert _err(lib, "kmoe_rmsnorm", FAKE, BF, FAKE, F32, 1e-5, 16, 8200, FAKE, FAKE, NULL, NULL, NULL)[0] == -6
    assert _err(lib, "kmoe_rmsnorm", FAKE, BF, FAKE, F32, -1.0, 16, 64, FAKE, FAKE, NULL, NULL, NULL)[0] == -2
    need = lib.kmoe_rmsnorm_bwd_workspace_bytes(5000, 64)
    assert need == -(-5000 // 24) * 64 * 4  # segments of 24 rows (a multiple of 8; at most 256 of them)
    rc, msg = _err(lib, "kmoe_rmsnorm_bwd", FAKE, FAKE, BF, FAKE, F32, FAKE, NULL, 5000, 64, FAKE, FAKE, BF, FAKE,
                   need - 4, NULL)
    assert rc == -4 and "workspace" in msg
    assert _err(lib, "kmoe_rmsnorm_bwd", FAKE, FAKE, BF, FAKE, F32, NULL, NULL, 16, 64, FAKE, FAKE, BF, FAKE, 1 << 20,
                NULL)[0] == -1
    assert _err(lib, "kmoe_mod_bwd", NULL, FAKE, 2, 8, FAKE, 64, FAKE, 1, NULL, BF, NULL, 0, NULL)[0] == -1
    assert _err(lib, "kmoe_mod_bwd", FAKE, FAKE, 0, 8, FAKE, 64, FAKE, 1, NULL, BF, NULL, 0, NULL)[0] == -2
    assert lib.kmoe_mod_bwd_workspace_bytes(1000, 64) == -(-1000 // 4) * 64 * 4
    assert _err(lib, "kmoe_combine_bwd_rows", FAKE, FAKE, FAKE, FAKE, 2, 12, 16, NULL, NULL, FAKE, FAKE, NULL,
                NULL)[0] == -2
    assert _err(lib, "kmoe_combine_bwd_rows", FAKE, FAKE, NULL, FAKE, 2, 64, 16, NULL, NULL, FAKE, FAKE, NULL,
                NULL)[0] == -1
