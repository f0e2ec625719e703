"""The C ABI library loads without a GPU, exports every entry point include/*.h declares with
the signatures the binding expects, and rejects bad arguments on the host (no GPU call)."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from mini_infra_qwen3_amd import _native

# These tests hand the library placeholder pointers that only a rejected call may see; where a
# device is visible a call that slipped past its checks would launch on them, so they run only
# without one (device_count does not initialise the runtime).
pytestmark = pytest.mark.skipif(torch.cuda.device_count() > 0, reason="host-only: placeholder pointers")

HEADERS = sorted((Path(__file__).resolve().parents[1] / "include").glob("*.h"))
DECL = re.compile(r"^\s*(?:const\s+)?[\w\s\*]+?\b(mi_\w+)\s*\(", re.M)


def declared_symbols() -> set[str]:
    names = set()
    for header in HEADERS:
        names.update(DECL.findall(header.read_text()))
    return names


def test_headers_declare_the_entry_points():
    names = declared_symbols()
    assert {"mi_abi_version", "mi_last_error", "mi_reshape_and_cache", "mi_gather_blocks",
            "mi_paged_decode_attention", "mi_paged_decode_workspace_bytes", "mi_chunked_prefill_attention"} <= names


def test_library_exports_every_declared_symbol(native_lib):
    for name in sorted(declared_symbols()):
        assert hasattr(native_lib, name), f"{name} declared in include/ but not exported"


def test_binding_covers_every_declared_symbol():
    assert declared_symbols() == set(_native.SIGNATURES)


def test_abi_version(native_lib):
    assert native_lib.mi_abi_version() == _native.ABI_VERSION


def test_decode_workspace_size(native_lib):
    # two slots per block range per head, (128 + 2) floats each; ranges = resident workgroups
    # (256 CUs x 4, over 4 head groups at 8 KV heads; 256 CUs assumed without a device), fewer
    # for launches under 16 blocks per range
    slot = 2 * 16 * 130 * 4
    assert native_lib.mi_paged_decode_workspace_bytes(256, 512, 16, 8, 128, 16) == 256 * slot
    assert native_lib.mi_paged_decode_workspace_bytes(256, 32, 16, 8, 128, 16) == 256 * slot
    assert native_lib.mi_paged_decode_workspace_bytes(4, 33, 16, 8, 128, 16) == 9 * slot
    assert native_lib.mi_paged_decode_workspace_bytes(16, 80, 16, 8, 128, 16) == 80 * slot
    assert native_lib.mi_paged_decode_workspace_bytes(1, 1, 16, 8, 128, 16) == 1 * slot
    assert native_lib.mi_paged_decode_workspace_bytes(0, 512, 16, 8, 128, 16) == 0
    assert native_lib.mi_paged_decode_workspace_bytes(8, 0, 16, 8, 128, 16) == 0
    # 2 KV heads: one head group, so ranges = 256 x 4
    assert native_lib.mi_paged_decode_workspace_bytes(512, 512, 4, 2, 128, 16) == 1024 * 2 * 4 * 130 * 4
    # GQA group 4 on 8 KV heads: the ranges follow the KV heads, the slots the 32 query heads
    assert native_lib.mi_paged_decode_workspace_bytes(256, 512, 32, 8, 128, 16) == 256 * 2 * 32 * 130 * 4
    assert native_lib.mi_paged_decode_workspace_bytes(256, 512, 16, 3, 128, 16) == 0  # heads not a multiple


def test_noalloc_decode_rejects_launches_beyond_its_scratch_on_host(native_lib):
    # 2 KV heads x 8 query heads each: 1024 block ranges (256 CUs assumed without a device) x 2
    # slots x 16 heads x 130 floats = 17 MB > the 8 MiB fixed array; rejected before any device call
    need = native_lib.mi_paged_decode_workspace_bytes(4096, 512, 16, 2, 128, 16)
    assert need > 8 << 20
    rc = native_lib.mi_paged_decode_attention_noalloc(None, 0, None, 0, 0, None, None, 1, None, 512, 512, None, 1,
                                                      4096, 16, 2, 128, 16, 1.0, None)
    assert rc == _native.MI_ERR_WORKSPACE and b"scratch" in native_lib.mi_last_error()
    assert native_lib.mi_paged_decode_attention_noalloc(None, 0, None, 0, 0, None, None, 1, None, 512, 0, None, 1,
                                                        0, 16, 8, 128, 16, 1.0, None) == _native.MI_OK


def _ptrs(n):
    return (ctypes.c_void_p * n)(*([16] * n))


def test_scatter_rejects_bad_arguments_on_host(native_lib):
    lib = native_lib
    rc = lib.mi_reshape_and_cache(_ptrs(1), _ptrs(1), 0, 0, 0, 0, 0, 0, None, None, None, 1, -1, 1, 1,
                                  _ptrs(1), _ptrs(1), 1, 16, 8, 128, 2, None)
    assert rc == _native.MI_ERR_INVALID_ARGUMENT and b"negative" in lib.mi_last_error()
    rc = lib.mi_reshape_and_cache(_ptrs(1), _ptrs(1), 0, 0, 0, 0, 0, 0, None, None, None, 1, 4, 1, 1,
                                  _ptrs(1), _ptrs(1), 1, 16, 8, 128, 2, None)
    assert rc == _native.MI_ERR_INVALID_ARGUMENT  # null slot_mapping
    rc = lib.mi_reshape_and_cache(_ptrs(1), _ptrs(1), 0, 0, 0, 0, 0, 0, None, None, 16, 1, 4, 1, 1,
                                  _ptrs(1), _ptrs(1), 1, 16, 8, 128, 3, None)
    assert rc == _native.MI_ERR_INVALID_ARGUMENT  # element size 3
    # nothing to do is success
    assert lib.mi_reshape_and_cache(None, None, 0, 0, 0, 0, 0, 0, None, None, None, 1, 0, 0, 0,
                                    None, None, 0, 0, 8, 128, 2, None) == _native.MI_OK


def test_gather_rejects_bad_arguments_on_host(native_lib):
    lib = native_lib
    rc = lib.mi_gather_blocks(_ptrs(1), _ptrs(1), 8, 16, 1, 2, 4, _ptrs(1), _ptrs(1), 1, 65536, None)
    assert rc == _native.MI_ERR_INVALID_ARGUMENT and b"stride" in lib.mi_last_error()
    rc = lib.mi_gather_blocks(_ptrs(1), _ptrs(1), 8, None, 4, 2, 4, _ptrs(1), _ptrs(1), 1, 65536, None)
    assert rc == _native.MI_ERR_INVALID_ARGUMENT


def test_decode_rejects_unsupported_shapes_on_host(native_lib):
    lib = native_lib
    args = dict(out=16, q=16, kp=16, vp=16, bt=16, ctx=16)

    def call(heads=16, kv=8, dim=128, bs=16, ws=None, ws_bytes=0, max_blocks=4):
        return lib.mi_paged_decode_attention(args["out"], heads * dim, args["q"], heads * dim, dim, args["kp"],
                                             args["vp"], 100, args["bt"], max_blocks, max_blocks, args["ctx"], 1,
                                             2, heads, kv, dim, bs, 0.1, ws, ws_bytes, None)

    assert call(dim=64) == _native.MI_ERR_UNSUPPORTED
    assert call(bs=8) == _native.MI_ERR_UNSUPPORTED
    assert call(heads=24) == _native.MI_ERR_UNSUPPORTED  # GQA group 3: no kernel compiled for it
    assert call(heads=20) == _native.MI_ERR_UNSUPPORTED  # not a multiple of the 8 KV heads
    assert call(heads=6, kv=3) == _native.MI_ERR_UNSUPPORTED
    assert call(max_blocks=40) == _native.MI_ERR_WORKSPACE  # no workspace
    assert b"workspace" in lib.mi_last_error()
    need = lib.mi_paged_decode_workspace_bytes(2, 40, 16, 8, 128, 16)
    assert call(max_blocks=40, ws=256, ws_bytes=need - 4) == _native.MI_ERR_WORKSPACE


def test_check_maps_status_to_python_errors(native_lib):
    native_lib.mi_gather_blocks(_ptrs(1), _ptrs(1), 8, None, 4, 2, 4, _ptrs(1), _ptrs(1), 1, 65536, None)
    with pytest.raises(ValueError, match="null pointer"):
        _native.check(_native.MI_ERR_INVALID_ARGUMENT, "x")
    with pytest.raises(RuntimeError):
        _native.check(_native.MI_ERR_DEVICE, "x")


def test_prefill_rejects_unsupported_shapes_on_host(native_lib):
    lib = native_lib

    def call(heads=16, kv=8, dim=128, bs=16, tok=128, nb=2, hist=16, hstride=2):
        return lib.mi_chunked_prefill_attention(16, 2048 * 4, 2048, 16, 16 * 4 * 128, 4 * 128, tok, 16, 8 * 4 * 128,
                                                4 * 128, tok, 16, 8 * 4 * 128, 4 * 128, tok, 16, 16, 100,
                                                hist, hstride, nb, 16, 16, 1, 2, 4, heads, kv, dim, bs, 0.1, None)

    assert call(dim=64) == _native.MI_ERR_UNSUPPORTED
    assert call(bs=32) == _native.MI_ERR_UNSUPPORTED
    assert call(heads=12) == _native.MI_ERR_UNSUPPORTED  # not a multiple of the 8 KV heads
    assert call(tok=100) == _native.MI_ERR_UNSUPPORTED  # stride not a multiple of 8 elements
    assert call(tok=1 << 24) == _native.MI_ERR_UNSUPPORTED  # key / value token stride >= 2^24 elements
    assert call(hstride=1) == _native.MI_ERR_INVALID_ARGUMENT
    assert call(hist=None) == _native.MI_ERR_INVALID_ARGUMENT
    assert call(nb=16385, hstride=16385) == _native.MI_ERR_UNSUPPORTED  # history table beyond 64 KiB of LDS


@pytest.mark.parametrize("exact", [False, True])
def test_mixed_attention_rejects_bad_arguments_on_host(native_lib, exact):
    entry = native_lib.mi_mixed_paged_attention_exact if exact else native_lib.mi_mixed_paged_attention

    def call(rows=2, width=64, decode=3, heads=16, kv=8, dim=128, bs=16, nb=4, hstride=4, mb=8, bstride=8,
             slots=16, tok=2048, chunk_tokens=0, chunk_first=None):
        return entry(16, 2048, 16, tok, 128, 16, 1024, 128, 16, 1024, 128, 16, 16, 100, rows, width, chunk_tokens,
                     chunk_first, 16, hstride, nb, 16, 16, 1, decode, 16, bstride, mb, 16, 1, slots, 1, heads, kv,
                     dim, bs, 0.1, None)

    assert call(dim=64) == _native.MI_ERR_UNSUPPORTED
    assert call(bs=32) == _native.MI_ERR_UNSUPPORTED
    assert call(heads=12) == _native.MI_ERR_UNSUPPORTED  # not a multiple of the 8 KV heads
    assert call(rows=-1) == _native.MI_ERR_INVALID_ARGUMENT
    assert call(decode=-2) == _native.MI_ERR_INVALID_ARGUMENT
    assert call(slots=None) == _native.MI_ERR_INVALID_ARGUMENT  # decode rows need their slots
    assert call(hstride=3) == _native.MI_ERR_INVALID_ARGUMENT
    assert call(bstride=7) == _native.MI_ERR_INVALID_ARGUMENT
    assert call(rows=70000) == _native.MI_ERR_UNSUPPORTED
    if exact:
        assert call(heads=24) == _native.MI_ERR_UNSUPPORTED  # GQA group 3: no exact kernel for it
    else:
        assert call(tok=100) == _native.MI_ERR_UNSUPPORTED  # stride not a multiple of 8 elements
    assert call(rows=0, decode=0) == _native.MI_OK  # nothing to do
    assert call(chunk_tokens=-1, chunk_first=16) == _native.MI_ERR_INVALID_ARGUMENT  # ragged rows, negative size


def test_argmax_rejects_bad_arguments_on_host(native_lib):
    lib = native_lib
    assert lib.mi_argmax_rows(16, 16, 4, 0, 16, None) == _native.MI_ERR_INVALID_ARGUMENT
    assert lib.mi_argmax_rows(16, 16, -1, 8, 8, None) == _native.MI_ERR_INVALID_ARGUMENT
    assert lib.mi_argmax_rows(16, 16, 2, 100, 99, None) == _native.MI_ERR_INVALID_ARGUMENT
    assert lib.mi_argmax_rows(None, 16, 2, 8, 8, None) == _native.MI_ERR_INVALID_ARGUMENT
    assert lib.mi_argmax_rows(None, None, 0, 8, 8, None) == _native.MI_OK
    assert lib.mi_argmax_rows(16, 16, 1 << 31, 8, 8, None) == _native.MI_ERR_UNSUPPORTED


def test_empty_pool_is_rejected_before_any_read_on_host(native_lib):
    """An out-of-range block id reads the null block 0, which a pool of no blocks lacks: every entry
    point that would read a block of such a pool refuses the call before any launch."""
    lib = native_lib
    bad = _native.MI_ERR_INVALID_ARGUMENT
    assert lib.mi_gather_blocks(_ptrs(1), _ptrs(1), 0, 16, 4, 2, 4, _ptrs(1), _ptrs(1), 1, 65536, None) == bad
    assert b"no blocks" in lib.mi_last_error()
    assert lib.mi_pack_blocks(16, _ptrs(1), _ptrs(1), 0, 16, 3, 1, 65536, None) == bad
    decode = lib.mi_paged_decode_attention(16, 2048, 16, 2048, 128, 16, 16, 0, 16, 4, 4, 16, 1, 2, 16, 8, 128, 16,
                                           0.1, None, 0, None)
    assert decode == bad
    noalloc = lib.mi_paged_decode_attention_noalloc(16, 2048, 16, 2048, 128, 16, 16, 0, 16, 4, 4, 16, 1, 2, 16, 8,
                                                    128, 16, 0.1, None)
    assert noalloc == bad
    exact = lib.mi_paged_decode_attention_exact(16, 2048, 16, 2048, 128, None, 0, None, 0, None, None, None, None,
                                                1e-6, None, 1, 16, 16, 0, 16, 4, 4, 16, 1, 2, 16, 8, 128, 16, 0.1,
                                                None, 0, None)
    assert exact == bad
    for entry in (lib.mi_chunked_prefill_attention, lib.mi_chunked_prefill_attention_exact):
        rc = entry(16, 2048 * 4, 2048, 16, 16 * 4 * 128, 4 * 128, 128, 16, 8 * 4 * 128, 4 * 128, 128, 16,
                   8 * 4 * 128, 4 * 128, 128, 16, 16, 0, 16, 2, 2, 16, 16, 1, 2, 4, 16, 8, 128, 16, 0.1, None)
        assert rc == bad
    for entry in (lib.mi_mixed_paged_attention, lib.mi_mixed_paged_attention_exact):
        rc = entry(16, 2048, 16, 2048, 128, 16, 1024, 128, 16, 1024, 128, 16, 16, 0, 0, 0, 0, None, None, 0, 0,
                   None, None, 1, 3, 16, 8, 8, 16, 1, 16, 1, 16, 8, 128, 16, 0.1, None)
        assert rc == bad


def test_exact_decode_split_workspace_size(native_lib):
    # launches of at most 48 (sequence, KV head) pairs split: splits = min(ceil(2 x 256 CUs / pairs),
    # 32, max_blocks / 4); fewer than 2 = unsplit (0)
    lib = native_lib
    assert lib.mi_paged_decode_exact_workspace_bytes(256, 512, 16, 8) == 0   # 2048 pairs fill the GPU
    assert lib.mi_paged_decode_exact_workspace_bytes(9, 72, 16, 8) == 0      # 72 pairs: one launch wins
    assert lib.mi_paged_decode_exact_workspace_bytes(4, 4, 16, 8) == 0       # one split per 4 blocks at most
    assert lib.mi_paged_decode_exact_workspace_bytes(0, 64, 16, 8) == 0
    # 6 sequences x 8 KV heads: 11 splits; scores 48 x 72 x 16 x 2 x 2 B (256-aligned), partials 48 x 11 x 2 x 128 x 8 B
    scores = -(-(48 * 72 * 16 * 2 * 2) // 256) * 256
    assert lib.mi_paged_decode_exact_workspace_bytes(6, 72, 16, 8) == scores + 48 * 11 * 2 * 128 * 8
    # one sequence: 32 splits (capped), GQA group 4
    assert lib.mi_paged_decode_exact_workspace_bytes(1, 200, 32, 8) == 8 * 200 * 16 * 4 * 2 + 8 * 32 * 4 * 128 * 8


def test_exact_decode_rejects_a_short_workspace_on_host(native_lib):
    lib = native_lib
    need = lib.mi_paged_decode_exact_workspace_bytes(2, 64, 16, 8)
    assert need > 0
    rc = lib.mi_paged_decode_attention_exact(16, 2048, 16, 2048, 128, None, 0, None, 0, None, None, None, None, 1e-6,
                                             None, 1, 16, 16, 100, 16, 64, 64, 16, 1, 2, 16, 8, 128, 16, 0.1, 256,
                                             need - 8, None)
    assert rc == _native.MI_ERR_WORKSPACE and b"split" in lib.mi_last_error()
    rc = lib.mi_paged_decode_attention_exact(16, 2048, 16, 2048, 128, None, 0, None, 0, None, None, None, None, 1e-6,
                                             None, 1, 16, 16, 100, 16, 64, 64, 16, 1, 2, 16, 8, 128, 16, 0.1, None,
                                             64, None)
    assert rc == _native.MI_ERR_INVALID_ARGUMENT
