"""C ABI checks that need no GPU: the library loads, exports every entry point
include/tmac_attn.h declares, and rejects calls without a context before
touching the device."""
import ctypes
import subprocess

import pytest

import tmac_attn


def test_library_loads_and_reports_version():
    lib = tmac_attn.load_library()
    assert lib.tmac_abi_version() == 1


def test_every_declared_symbol_is_exported():
    declared = tmac_attn.declared_symbols()
    assert len(declared) >= 30
    out = subprocess.run(["nm", "-D", "--defined-only", tmac_attn.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    # and the Python front end binds exactly the declared set
    assert sorted(tmac_attn.SIGNATURES) == declared


def test_status_strings():
    assert tmac_attn.status_string(0) == "ok"
    assert "unsupported" in tmac_attn.status_string(tmac_attn.TMAC_ERR_UNSUPPORTED)
    assert tmac_attn.status_string(424242) == "unknown status" or tmac_attn.status_string(424242)


def test_calls_without_context_are_rejected():
    lib = tmac_attn.load_library()
    nc = tmac_attn.TMAC_ERR_NOT_INITIALIZED
    assert lib.tmac_attention_op(None, None, 16, 16, 16, 16, 14, 2, 64, 0) == nc
    assert lib.tmac_rope_op(None, None, 16, 14, 64, 0, 1e6) == nc
    assert lib.tmac_elem_op(None, None, 2, 16, 16, 128) == nc
    assert lib.tmac_layer_attention(None, None, 16, 16, 16, 16, 16, 16, 14, 2, 64, 0, 256, 1e6) == nc
    assert lib.tmac_attention_decode_batched(None, None, 16, 16, 16, 16, 1, 14, 2, 64, 1, 1) == nc
    assert lib.tmac_attention_decode_ragged(None, None, 16, 16, 16, 16, 16, 16, 1, 14, 2, 64, 1, 0) == nc
    assert lib.tmac_prefill_pack_rows(None, None, 0, 16, 16, 16, 16, 16, 1, 2, 64, 0, 1) == nc
    assert lib.tmac_attention_prefill_tiles(None, None, 16, 16, 16, 16, 1, 1, 0, 14, 2, 64) == nc
    assert lib.tmac_step_begin(None, None) == nc
    assert lib.tmac_malloc(None, ctypes.byref(ctypes.c_void_p()), 16) == nc
    assert lib.tmac_shutdown(None) == nc



# Entry points whose first argument is not a live context by design: the model
# functions take a model handle (a model may be loaded without a context), and a
# graph may be destroyed after its context is shut down.
NO_CONTEXT = {"tmac_status_string", "tmac_last_error", "tmac_abi_version", "tmac_init", "tmac_synth_normal",
              "tmac_synth_uniform", "tmac_prefill_tiles_bytes", "tmac_model_load", "tmac_model_count",
              "tmac_model_tensor", "tmac_model_find", "tmac_model_free", "tmac_graph_destroy"}


def _null_args(argtypes):
    return [0.0 if a in (ctypes.c_float, ctypes.c_double)
            else 0 if a in (ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_uint64)
            else None for a in argtypes]


def test_every_context_entry_point_rejects_a_null_context():
    """Every entry point that takes a context returns TMAC_ERR_NOT_INITIALIZED for a
    null one (every other argument null or zero), before it reads any argument."""
    lib = tmac_attn.load_library()
    checked = []
    for name, (_, argtypes) in tmac_attn.SIGNATURES.items():
        if name in NO_CONTEXT:
            continue
        assert argtypes and argtypes[0] is ctypes.c_void_p, name
        assert getattr(lib, name)(*_null_args(argtypes)) == tmac_attn.TMAC_ERR_NOT_INITIALIZED, name
        checked.append(name)
    assert len(checked) >= 40


def test_context_free_entry_points_on_null_handles():
    """The documented exceptions: destroying a null graph or freeing a null model is a
    no-op; the model queries report a null handle."""
    lib = tmac_attn.load_library()
    assert lib.tmac_graph_destroy(None, None) == tmac_attn.TMAC_OK
    assert lib.tmac_model_free(None, None) == tmac_attn.TMAC_OK
    assert lib.tmac_model_count(None) < 0
    assert lib.tmac_model_load(None, None, None) == tmac_attn.TMAC_ERR_NULL_POINTER
    assert lib.tmac_model_tensor(None, 0, None) == tmac_attn.TMAC_ERR_NULL_POINTER
    assert lib.tmac_model_find(None, None, None) == tmac_attn.TMAC_ERR_NULL_POINTER

def test_prefill_tiles_bytes():
    """16 KiB per 64-row tile and (sequence, kv head); rows rounded up to whole 4-tile stages."""
    lib = tmac_attn.load_library()
    tile = 2 * 64 * 64 * 2
    assert lib.tmac_prefill_tiles_bytes(4, 2, 2048) == 4 * 2 * 32 * tile
    assert lib.tmac_prefill_tiles_bytes(1, 1, 1) == 4 * tile
    assert lib.tmac_prefill_tiles_bytes(1, 2, 257) == 2 * 8 * tile
    assert lib.tmac_prefill_tiles_bytes(0, 2, 100) == 0
    assert lib.tmac_prefill_tiles_bytes(1, 0, 100) == 0 and lib.tmac_prefill_tiles_bytes(1, 2, 0) == 0


def test_init_without_gpu_fails_cleanly():
    """In a container without a GPU, tmac_init must fail with a HIP status, not crash
    or fall back to the CPU."""
    lib = tmac_attn.load_library()
    h = ctypes.c_void_p()
    rc = lib.tmac_init(ctypes.byref(h), 0)
    if rc == tmac_attn.TMAC_OK:  # running on a GPU box
        lib.tmac_shutdown(h)
        pytest.skip("a GPU is present")
    assert rc >= tmac_attn.TMAC_ERR_HIP_BASE or rc in (tmac_attn.TMAC_ERR_INVALID_ARG,
                                                      tmac_attn.TMAC_ERR_UNSUPPORTED)
    assert h.value is None
