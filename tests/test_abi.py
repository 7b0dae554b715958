"""The C ABI of libmk.so, checked on the CPU (no GPU calls are made).

* the library loads and exports every function include/mk.h declares;
* argument validation rejects bad requests with the documented error codes
  before touching the HIP runtime (the reference only had Python asserts on
  shapes and TP degree, llama_with_megakernel.py:145-162; this ABI returns a
  code and a message instead of launching).
"""

import ctypes
from ctypes import POINTER, c_void_p

import pytest

from conftest import REPO


@pytest.fixture(scope="module")
def lib():
    import mk_lib
    if not mk_lib.LIB_PATH.exists():
        import build_lib
        build_lib.build()
    return mk_lib.load()


def test_exports_every_declared_function(lib):
    import mk_lib
    names = mk_lib.header_functions(REPO / "include" / "mk.h")
    assert set(names) >= {"mk_decode_step", "mk_layer_step", "mk_workspace_bytes", "mk_workspace_init",
                          "mk_read_device_error", "mk_last_error", "mk_abi_version", "mk_grid_size"}
    for n in names:
        assert hasattr(lib, n), n
    assert lib.mk_abi_version() == 1


def test_workspace_size(lib):
    assert lib.mk_workspace_bytes(1, 1024) > 0
    assert lib.mk_workspace_bytes(1, 8192) >= lib.mk_workspace_bytes(1, 1024)
    assert lib.mk_workspace_bytes(0, 1024) == 0
    assert lib.mk_workspace_bytes(1, 0) == 0
    # batched layouts (2..32 sequences): larger batches need more, 33 is unsupported
    sizes = [lib.mk_workspace_bytes(b, 4096) for b in range(1, 33)]
    assert all(s > 0 for s in sizes)
    assert sizes == sorted(sizes) and sizes[1] > sizes[0]
    assert lib.mk_workspace_bytes(33, 4096) == 0


def _args(**over):
    import mk_lib
    kc = (c_void_p * 16)(*([0x1000] * 16))
    vc = (c_void_p * 16)(*([0x2000] * 16))
    a = dict(first_layer=0, n_layers=16, batch=1, s_max=1024,
             k_cache=ctypes.cast(kc, POINTER(c_void_p)), v_cache=ctypes.cast(vc, POINTER(c_void_p)),
             tokens=0x3000, hidden_in=None, pos=0x4000, hidden_out=None, logits=None, next_token=0x5000,
             flags=0, workspace=0x100000, workspace_bytes=1 << 24, stream=None)
    a.update(over)
    keep = (kc, vc)
    return mk_lib.MkStepArgs(**a), keep


def _weights(**over):
    import mk_lib
    w = dict(w_qkv=0x10000, w_o=0x20000, w_gu=0x30000, w_down=0x40000, embed=0x50000,
             norm_final=0x60000, rope=0x70000, n_layers=16, rope_rows=8192)
    w.update(over)
    return mk_lib.MkWeights(**w)


@pytest.mark.parametrize("over,code", [
    (dict(n_layers=0), -2),
    (dict(n_layers=17), -2),
    (dict(first_layer=15, n_layers=2), -2),
    (dict(batch=0), -2),
    (dict(batch=33), -2),
    (dict(s_max=0), -2),
    (dict(s_max=9000), -2),
    (dict(tokens=None), -1),
    (dict(hidden_in=0x9000), -1),
    (dict(pos=None), -1),
    (dict(workspace=None), -1),
    (dict(workspace=0x100010), -3),
    (dict(workspace_bytes=100), -3),
    (dict(k_cache=None), -1),
])
def test_rejects_bad_arguments(lib, over, code):
    a, keep = _args(**over)
    w = _weights()
    rc = lib.mk_decode_step(ctypes.byref(w), ctypes.byref(a))
    assert rc == code, (rc, lib.mk_last_error())
    assert lib.mk_last_error()


def test_rejects_bad_weights(lib):
    a, keep = _args()
    assert lib.mk_decode_step(ctypes.byref(_weights(w_o=None)), ctypes.byref(a)) == -1
    assert lib.mk_decode_step(ctypes.byref(_weights(w_o=0x20008)), ctypes.byref(a)) == -7
    assert lib.mk_decode_step(ctypes.byref(_weights(n_layers=8)), ctypes.byref(a)) == -2
    assert lib.mk_decode_step(None, ctypes.byref(a)) == -1


def test_rejects_null_cache_entry(lib):
    import mk_lib
    kc = (c_void_p * 16)(*([0x1000] * 15 + [None]))
    a, keep = _args(k_cache=ctypes.cast(kc, POINTER(c_void_p)))
    assert lib.mk_decode_step(ctypes.byref(_weights()), ctypes.byref(a)) == -1


def test_layer_step_requires_hidden(lib):
    w = _weights()
    rc = lib.mk_layer_step(ctypes.byref(w), 0, 1, 1024, 0x1000, 0x2000, None, 0x4000, 0x5000, 0x100000,
                           1 << 24, None)
    assert rc == -1


def test_workspace_release_requires_workspace(lib):
    assert lib.mk_workspace_release(None) == -1
    assert b"NULL" in lib.mk_last_error()


def test_noalloc_step_argument_checks(lib):
    """mk_decode_step_noalloc: batch 1 only, no prefill, no workspace (checked before any HIP call)."""
    w = _weights()
    a, keep = _args(workspace=None, workspace_bytes=0, batch=2)
    assert lib.mk_decode_step_noalloc(ctypes.byref(w), ctypes.byref(a)) == -2
    assert b"batch 1" in lib.mk_last_error()
    a, keep = _args(workspace=None, workspace_bytes=0, flags=4)
    assert lib.mk_decode_step_noalloc(ctypes.byref(w), ctypes.byref(a)) == -4
    a, keep = _args()
    assert lib.mk_decode_step_noalloc(ctypes.byref(w), ctypes.byref(a)) == -3
    a, keep = _args(workspace=None, workspace_bytes=0, pos=None)
    assert lib.mk_decode_step_noalloc(ctypes.byref(w), ctypes.byref(a)) == -1


def test_decode_loop_argument_checks(lib):
    """mk_decode_loop: n_steps in [1, 2^20], batch 1, token input, the final
    norm's weights (every step runs the lm_head), aligned outputs; all checked
    before any HIP call."""
    w = _weights()
    a, keep = _args()
    assert lib.mk_decode_loop(ctypes.byref(w), ctypes.byref(a), 0, None, None) == -2
    assert lib.mk_decode_loop(ctypes.byref(w), ctypes.byref(a), (1 << 20) + 1, None, None) == -2
    a, keep = _args(batch=2)
    assert lib.mk_decode_loop(ctypes.byref(w), ctypes.byref(a), 4, None, None) == -4
    a, keep = _args(next_token=None)
    assert lib.mk_decode_loop(ctypes.byref(_weights(norm_final=None)), ctypes.byref(a), 4, None, None) == -1
    assert b"norm_final" in lib.mk_last_error()
    a, keep = _args()
    assert lib.mk_decode_loop(ctypes.byref(w), ctypes.byref(a), 4, 0x9001, None) == -7
    assert lib.mk_decode_loop(ctypes.byref(w), ctypes.byref(a), 4, None, 0x9008) == -7


def _pf_args(**over):
    import mk_lib
    kc = (c_void_p * 16)(*([0x1000] * 16))
    vc = (c_void_p * 16)(*([0x2000] * 16))
    a = dict(first_layer=0, n_layers=16, n_tokens=100, start_pos=0, s_max=1024, tokens=0x3000,
             k_cache=ctypes.cast(kc, POINTER(c_void_p)), v_cache=ctypes.cast(vc, POINTER(c_void_p)),
             hidden_out=None, workspace=0x100000, workspace_bytes=1 << 24, stream=None)
    a.update(over)
    return mk_lib.MkPrefillArgs(**a), (kc, vc)


def test_prefill_workspace_size(lib):
    """mk_prefill_workspace_bytes: linear in the chunk (multiples of 16 tokens), 0 outside [1, 16384]."""
    assert lib.mk_prefill_workspace_bytes(0) == 0
    assert lib.mk_prefill_workspace_bytes(16385) == 0
    assert lib.mk_prefill_workspace_bytes(1) == lib.mk_prefill_workspace_bytes(16)
    b16, b32 = lib.mk_prefill_workspace_bytes(16), lib.mk_prefill_workspace_bytes(32)
    per_token = (b32 - b16) // 16
    assert per_token == 2048 * 2 * 5 + 8192 * 2          # x, h1, q, xn, att (bf16 [2048]) + act (bf16 [8192])
    assert lib.mk_prefill_workspace_bytes(4096) == b16 + (4096 - 16) * per_token


@pytest.mark.parametrize("over,code", [
    (dict(n_layers=0), -2),
    (dict(first_layer=15, n_layers=2), -2),
    (dict(n_tokens=0), -2),
    (dict(start_pos=-1), -2),
    (dict(start_pos=1000, n_tokens=25), -2),      # past s_max
    (dict(s_max=9000), -2),                       # beyond the RoPE table
    (dict(tokens=None), -1),
    (dict(k_cache=None), -1),
    (dict(workspace=None), -1),
    (dict(workspace=0x100010), -3),
    (dict(workspace_bytes=1000), -3),
    (dict(tokens=0x3004), -7),
])
def test_prefill_rejects_bad_arguments(lib, over, code):
    a, keep = _pf_args(**over)
    rc = lib.mk_prefill(ctypes.byref(_weights()), ctypes.byref(a))
    assert rc == code, (rc, lib.mk_last_error())
    assert lib.mk_last_error()


def test_prefill_rejects_bad_weights(lib):
    a, keep = _pf_args()
    assert lib.mk_prefill(ctypes.byref(_weights(w_gu=None)), ctypes.byref(a)) == -1
    assert lib.mk_prefill(ctypes.byref(_weights(n_layers=8)), ctypes.byref(a)) == -2
    assert lib.mk_prefill(None, ctypes.byref(a)) == -1
