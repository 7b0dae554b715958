"""ctypes binding of ``libmk.so`` (declared in ``include/mk.h``) and a small
device-state holder used by the Python seams.

This is the only module that talks to the native library. The library must be
built (``build_lib.py``); if it is missing, ``load()`` raises — there is no
fallback implementation of the decode step.
"""

from __future__ import annotations

import ctypes
import sys
import weakref
from ctypes import POINTER, c_char_p, c_int, c_int32, c_size_t, c_uint32, c_void_p
from pathlib import Path
from typing import Dict, List, Optional, Sequence

import torch

LIB_PATH = Path(__file__).resolve().with_name("libmk.so")
ABI_VERSION = 1             # MK_ABI_VERSION of include/mk.h

MK_OK = 0
ERRORS = {
    -1: "MK_ERR_NULL", -2: "MK_ERR_SHAPE", -3: "MK_ERR_WORKSPACE", -4: "MK_ERR_UNSUPPORTED",
    -5: "MK_ERR_HIP", -6: "MK_ERR_DEVICE", -7: "MK_ERR_ALIGN",
}
MK_DEVERR_POS = 0x1
MK_DEVERR_SYNC = 0x2
MK_DEVERR_BARRIER = MK_DEVERR_SYNC
MK_DEVERR_PREFILL = 0x4
MK_FLAG_ADVANCE = 0x1
MK_FLAG_COOPERATIVE = 0x2
MK_FLAG_PREFILL = 0x4
PREFILL_CHUNK = 32          # tokens per prefill step (the batched kernel's largest batch)

HIDDEN, N_KV, HEAD_DIM, VOCAB, MAX_LAYERS = 2048, 8, 64, 128256, 16


class MkWeights(ctypes.Structure):
    _fields_ = [
        ("w_qkv", c_void_p), ("w_o", c_void_p), ("w_gu", c_void_p), ("w_down", c_void_p),
        ("embed", c_void_p), ("norm_final", c_void_p), ("rope", c_void_p),
        ("n_layers", c_int32), ("rope_rows", c_int32),
        ("t_qkv", c_void_p), ("t_o", c_void_p), ("t_gu", c_void_p), ("t_down", c_void_p), ("t_embed", c_void_p),
    ]


TILED_KEYS = {"t_qkv": "w_qkv", "t_o": "w_o", "t_gu": "w_gu", "t_down": "w_down", "t_embed": "embed"}


class MkStepArgs(ctypes.Structure):
    _fields_ = [
        ("first_layer", c_int32), ("n_layers", c_int32), ("batch", c_int32), ("s_max", c_int32),
        ("k_cache", POINTER(c_void_p)), ("v_cache", POINTER(c_void_p)),
        ("tokens", c_void_p), ("hidden_in", c_void_p), ("pos", c_void_p),
        ("hidden_out", c_void_p), ("logits", c_void_p), ("next_token", c_void_p),
        ("flags", c_uint32), ("workspace", c_void_p), ("workspace_bytes", c_size_t),
        ("stream", c_void_p), ("trace", c_void_p),
    ]


class MkPrefillArgs(ctypes.Structure):
    _fields_ = [
        ("first_layer", c_int32), ("n_layers", c_int32), ("n_tokens", c_int32), ("start_pos", c_int32),
        ("s_max", c_int32), ("tokens", c_void_p), ("k_cache", POINTER(c_void_p)), ("v_cache", POINTER(c_void_p)),
        ("hidden_out", c_void_p), ("workspace", c_void_p), ("workspace_bytes", c_size_t), ("stream", c_void_p),
    ]


class MkSampleArgs(ctypes.Structure):
    _fields_ = [
        ("logits", c_void_p), ("batch", c_int32), ("vocab", c_int32), ("vocab_stride", c_int32),
        ("params", c_void_p), ("seed", ctypes.c_uint64), ("counter", c_void_p), ("tokens_out", c_void_p),
        ("uniforms_out", c_void_p), ("stream", c_void_p),
    ]


SAMPLE_MAX_TOPK = 1024


class MkError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{ERRORS.get(code, code)}: {msg}")
        self.code = code


_lib = None


def load() -> ctypes.CDLL:
    """Load libmk.so (raises FileNotFoundError if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(f"{LIB_PATH} is missing: build it with build_lib.py")
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.mk_abi_version.restype = c_int
        lib.mk_last_error.restype = c_char_p
        lib.mk_grid_size.argtypes = [c_int]
        lib.mk_grid_size.restype = c_int
        lib.mk_set_grid_size.argtypes = [c_int, c_int]
        lib.mk_set_grid_size.restype = c_int
        lib.mk_wall_clock_hz.argtypes = [c_int]
        lib.mk_wall_clock_hz.restype = ctypes.c_longlong
        lib.mk_workspace_bytes.argtypes = [c_int32, c_int32]
        lib.mk_workspace_bytes.restype = c_size_t
        lib.mk_workspace_init.argtypes = [c_void_p, c_size_t, c_void_p]
        lib.mk_workspace_init.restype = c_int
        lib.mk_workspace_release.argtypes = [c_void_p]
        lib.mk_workspace_release.restype = c_int
        lib.mk_read_device_error.argtypes = [c_void_p, c_void_p, POINTER(c_uint32)]
        lib.mk_read_device_error.restype = c_int
        lib.mk_decode_step.argtypes = [POINTER(MkWeights), POINTER(MkStepArgs)]
        lib.mk_decode_step.restype = c_int
        lib.mk_decode_loop.argtypes = [POINTER(MkWeights), POINTER(MkStepArgs), c_int32, c_void_p, c_void_p]
        lib.mk_decode_loop.restype = c_int
        lib.mk_decode_step_noalloc.argtypes = [POINTER(MkWeights), POINTER(MkStepArgs)]
        lib.mk_decode_step_noalloc.restype = c_int
        lib.mk_layer_step.argtypes = [POINTER(MkWeights), c_int32, c_int32, c_int32, c_void_p, c_void_p,
                                      c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]
        lib.mk_layer_step.restype = c_int
        lib.mk_prefill.argtypes = [POINTER(MkWeights), POINTER(MkPrefillArgs)]
        lib.mk_prefill.restype = c_int
        lib.mk_prefill_workspace_bytes.argtypes = [c_int32]
        lib.mk_prefill_workspace_bytes.restype = c_size_t
        lib.mk_sample.argtypes = [POINTER(MkSampleArgs)]
        lib.mk_sample.restype = c_int
        lib.mk_sample_last_error.restype = c_char_p
        if lib.mk_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI version {lib.mk_abi_version()}, this module {ABI_VERSION}: "
                               "rebuild it")
        _lib = lib
    return _lib


def check(rc: int) -> None:
    if rc != MK_OK:
        raise MkError(rc, load().mk_last_error().decode(errors="replace"))


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def current_stream_ptr() -> int:
    return torch.cuda.current_stream().cuda_stream


def weights_struct(packed: Dict[str, torch.Tensor], tiled: bool = True) -> MkWeights:
    """MkWeights view of ``mk_weights.pack_for_megakernel`` output (device tensors).
    The MFMA-tiled copies (``t_*``, read by the batched kernel) are passed when
    all five are present and ``tiled`` is true; otherwise the batched kernel
    reads the row-major stacks."""
    for k in ("w_qkv", "w_o", "w_gu", "w_down", "embed", "norm_final", "rope"):
        t = packed[k]
        if t.dtype != torch.bfloat16 or not t.is_contiguous():
            raise ValueError(f"{k} must be contiguous bf16")
    t_ptrs = [None] * 5
    if tiled and all(k in packed for k in TILED_KEYS):
        for k, src in TILED_KEYS.items():
            t = packed[k]
            if t.dtype != torch.bfloat16 or not t.is_contiguous() or t.numel() != packed[src].numel():
                raise ValueError(f"{k} must be a contiguous bf16 tiling of {src}")
        t_ptrs = [_ptr(packed[k]) for k in TILED_KEYS]
    return MkWeights(
        _ptr(packed["w_qkv"]), _ptr(packed["w_o"]), _ptr(packed["w_gu"]), _ptr(packed["w_down"]),
        _ptr(packed["embed"]), _ptr(packed["norm_final"]), _ptr(packed["rope"]),
        int(packed["w_qkv"].shape[0]), int(packed["rope"].shape[0]), *t_ptrs)


_deferred: List["_Released"] = []     # collected workspaces whose exchange area is not yet returned


def _drain_deferred() -> None:
    """Return the exchange areas of workspaces collected since the last call
    (never from a finaliser: mk_workspace_release synchronises the device,
    which is illegal while any stream captures a graph)."""
    while _deferred:
        ws = _deferred.pop()
        try:
            with torch.cuda.device(ws.device):
                check(load().mk_workspace_release(ws.buf.data_ptr()))
        except Exception:
            pass


class _Released:
    """A collected workspace's device and buffer, kept until its area is returned."""

    def __init__(self, device, buf):
        self.device, self.buf = device, buf


class Workspace:
    """Device workspace for one stream of steps (initialised once at creation).

    Its exchange area in the library is returned by ``release()``, which
    synchronises the device. A HIP graph that captured steps on this workspace
    holds the area's address in its kernel arguments, so ``release()`` refuses
    while a graph registered with ``register_graph`` is alive (a replay would
    write freed memory), and it must not be called during a stream capture.
    When the object is collected, its buffer and area are kept and returned by
    the next ``Workspace`` created, outside any capture."""

    def __init__(self, batch: int, s_max: int, device: torch.device):
        lib = load()
        _drain_deferred()
        n = lib.mk_workspace_bytes(batch, s_max)
        if n == 0:
            raise MkError(-4, f"no workspace size for batch={batch}, s_max={s_max}")
        self.nbytes = (n + 255) // 256 * 256
        self.device = torch.device(device)
        # torch's caching allocator returns 512-byte aligned blocks
        self.buf = torch.empty(self.nbytes, dtype=torch.uint8, device=device)
        assert self.buf.data_ptr() % 256 == 0
        self._live = False
        self._graphs = weakref.WeakSet()
        check(lib.mk_workspace_init(self.buf.data_ptr(), self.nbytes, c_void_p(current_stream_ptr())))
        self._live = True

    def register_graph(self, graph) -> None:
        """Record a graph that captured steps on this workspace: release()
        refuses while it is alive."""
        self._graphs.add(graph)

    def release(self) -> None:
        """mk_workspace_release: synchronises the device and returns the
        exchange area (the workspace is unusable afterwards)."""
        if not self._live:
            return
        if len(self._graphs):
            raise RuntimeError(f"{len(self._graphs)} HIP graph(s) that captured steps on this workspace are alive: "
                               "destroy them before releasing it")
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("a workspace cannot be released during stream capture")
        self._live = False
        with torch.cuda.device(self.device):
            check(load().mk_workspace_release(self.buf.data_ptr()))

    def __del__(self, _finalizing=sys.is_finalizing):
        if getattr(self, "_live", False) and not _finalizing():
            # no device synchronisation from a finaliser (it may run during a capture):
            # the next Workspace returns the area
            self._live = False
            _deferred.append(_Released(self.device, self.buf))

    def read_device_error(self) -> int:
        bits = c_uint32(0)
        check(load().mk_read_device_error(self.buf.data_ptr(), c_void_p(current_stream_ptr()),
                                          ctypes.byref(bits)))
        return bits.value


def decode_step(weights: MkWeights, ws: Workspace, k_caches: Sequence[torch.Tensor],
                v_caches: Sequence[torch.Tensor], pos: torch.Tensor, *,
                tokens: Optional[torch.Tensor] = None, hidden_in: Optional[torch.Tensor] = None,
                hidden_out: Optional[torch.Tensor] = None, logits: Optional[torch.Tensor] = None,
                next_token: Optional[torch.Tensor] = None, first_layer: int = 0,
                n_layers: Optional[int] = None, flags: int = 0, batch: int = 1,
                trace: Optional[torch.Tensor] = None) -> None:
    """One call of ``mk_decode_step`` on the current torch stream."""
    n = len(k_caches) if n_layers is None else n_layers
    if len(k_caches) < n or len(v_caches) < n:
        raise ValueError("need one K and one V cache per layer run")
    s_max = int(k_caches[0].shape[-2])
    kc = (c_void_p * n)(*[t.data_ptr() for t in k_caches[:n]])
    vc = (c_void_p * n)(*[t.data_ptr() for t in v_caches[:n]])
    a = MkStepArgs(first_layer, n, batch, s_max, ctypes.cast(kc, POINTER(c_void_p)),
                   ctypes.cast(vc, POINTER(c_void_p)), _ptr(tokens), _ptr(hidden_in), _ptr(pos),
                   _ptr(hidden_out), _ptr(logits), _ptr(next_token), flags, ws.buf.data_ptr(), ws.nbytes,
                   current_stream_ptr(), _ptr(trace))
    check(load().mk_decode_step(ctypes.byref(weights), ctypes.byref(a)))


def decode_loop(weights: MkWeights, ws: Workspace, k_caches: Sequence[torch.Tensor],
                v_caches: Sequence[torch.Tensor], pos: torch.Tensor, tokens: torch.Tensor, n_steps: int, *,
                tokens_out: Optional[torch.Tensor] = None, step_clock: Optional[torch.Tensor] = None,
                logits: Optional[torch.Tensor] = None, next_token: Optional[torch.Tensor] = None,
                hidden_out: Optional[torch.Tensor] = None, flags: int = 0) -> None:
    """``mk_decode_loop`` on the current torch stream: ``n_steps`` greedy batch-1
    decode steps in one launch (tokens_out: int32 [n_steps]; step_clock:
    int64 [n_steps + 1] device wall-clock ticks at the step boundaries)."""
    n = len(k_caches)
    kc = (c_void_p * n)(*[t.data_ptr() for t in k_caches])
    vc = (c_void_p * n)(*[t.data_ptr() for t in v_caches])
    a = MkStepArgs(0, n, 1, int(k_caches[0].shape[-2]), ctypes.cast(kc, POINTER(c_void_p)),
                   ctypes.cast(vc, POINTER(c_void_p)), _ptr(tokens), None, _ptr(pos), _ptr(hidden_out), _ptr(logits),
                   _ptr(next_token), flags, ws.buf.data_ptr(), ws.nbytes, current_stream_ptr(), None)
    check(load().mk_decode_loop(ctypes.byref(weights), ctypes.byref(a), int(n_steps), _ptr(tokens_out),
                                _ptr(step_clock)))


def decode_step_noalloc(weights: MkWeights, k_caches: Sequence[torch.Tensor], v_caches: Sequence[torch.Tensor],
                        pos: torch.Tensor, *, tokens: Optional[torch.Tensor] = None,
                        hidden_in: Optional[torch.Tensor] = None, hidden_out: Optional[torch.Tensor] = None,
                        logits: Optional[torch.Tensor] = None, next_token: Optional[torch.Tensor] = None,
                        first_layer: int = 0, n_layers: Optional[int] = None, flags: int = 0) -> None:
    """One call of ``mk_decode_step_noalloc`` (batch 1, no workspace: the
    library's static scratch) on the current torch stream."""
    n = len(k_caches) if n_layers is None else n_layers
    if len(k_caches) < n or len(v_caches) < n:
        raise ValueError("need one K and one V cache per layer run")
    kc = (c_void_p * n)(*[t.data_ptr() for t in k_caches[:n]])
    vc = (c_void_p * n)(*[t.data_ptr() for t in v_caches[:n]])
    a = MkStepArgs(first_layer, n, 1, int(k_caches[0].shape[-2]), ctypes.cast(kc, POINTER(c_void_p)),
                   ctypes.cast(vc, POINTER(c_void_p)), _ptr(tokens), _ptr(hidden_in), _ptr(pos),
                   _ptr(hidden_out), _ptr(logits), _ptr(next_token), flags, None, 0, current_stream_ptr(), None)
    check(load().mk_decode_step_noalloc(ctypes.byref(weights), ctypes.byref(a)))


PREFILL_MAX_CHUNK = 16384   # tokens one pass of mk_prefill's layer loop takes at most


def prefill_workspace(chunk_tokens: int, device) -> torch.Tensor:
    """A workspace for ``mk_prefill`` in chunks of up to ``chunk_tokens`` tokens
    (256-byte aligned device bytes)."""
    n = load().mk_prefill_workspace_bytes(min(max(int(chunk_tokens), 16), PREFILL_MAX_CHUNK))
    if n == 0:
        raise MkError(-2, f"no prefill workspace size for {chunk_tokens} tokens")
    buf = torch.empty(n, dtype=torch.uint8, device=device)
    assert buf.data_ptr() % 256 == 0
    return buf


def prefill(weights: MkWeights, tokens: torch.Tensor, k_caches: Sequence[torch.Tensor],
            v_caches: Sequence[torch.Tensor], start_pos: int, workspace: torch.Tensor, *,
            hidden_out: Optional[torch.Tensor] = None, first_layer: int = 0,
            n_layers: Optional[int] = None) -> None:
    """``mk_prefill`` on the current stream: the K/V rows of ``tokens`` (device
    int32 [T]) at positions start_pos .. start_pos + T - 1 of one sequence's
    caches (bf16 [8][S][64] or [1][8][S][64] per layer)."""
    n = len(k_caches) if n_layers is None else n_layers
    if len(k_caches) < n or len(v_caches) < n:
        raise ValueError("need one K and one V cache per layer run")
    if tokens.dtype != torch.int32 or not tokens.is_contiguous():
        raise ValueError("tokens must be contiguous int32")
    kc = (c_void_p * n)(*[t.data_ptr() for t in k_caches[:n]])
    vc = (c_void_p * n)(*[t.data_ptr() for t in v_caches[:n]])
    a = MkPrefillArgs(first_layer, n, int(tokens.numel()), int(start_pos), int(k_caches[0].shape[-2]),
                      tokens.data_ptr(), ctypes.cast(kc, POINTER(c_void_p)), ctypes.cast(vc, POINTER(c_void_p)),
                      _ptr(hidden_out), workspace.data_ptr(), workspace.numel(), current_stream_ptr())
    check(load().mk_prefill(ctypes.byref(weights), ctypes.byref(a)))


def set_grid_size(workgroups: int, device: Optional[int] = None) -> None:
    """``mk_set_grid_size``: run the kernels on ``workgroups`` workgroups (0:
    one per CU) for the steps launched after the call."""
    dev = torch.cuda.current_device() if device is None else device
    check(load().mk_set_grid_size(dev, workgroups))


def grid_size(device: Optional[int] = None) -> int:
    dev = torch.cuda.current_device() if device is None else device
    g = load().mk_grid_size(dev)
    if g < 0:
        check(g)
    return g


def noalloc_device_error() -> int:
    """Sticky device error bits of every faulted ``mk_decode_step_noalloc``
    step on the current device since the last call (returned and cleared)."""
    bits = c_uint32(0)
    check(load().mk_read_device_error(None, c_void_p(current_stream_ptr()), ctypes.byref(bits)))
    return bits.value


def prepare_sampling_params(batch_size: int, top_k, top_p, temperature, device="cuda") -> torch.Tensor:
    """Device fp32 [batch][3] rows (top_k, top_p, temperature); a single value
    broadcasts (the tensor NxDI's prepare_sampling_params builds, main.py:195-206)."""
    def col(v):
        v = list(v) if isinstance(v, (list, tuple)) else [v]
        return v * batch_size if len(v) == 1 else v
    rows = list(zip(col(top_k), col(top_p), col(temperature)))
    if len(rows) != batch_size:
        raise ValueError(f"sampling parameters for {len(rows)} rows, batch {batch_size}")
    return torch.tensor(rows, dtype=torch.float32, device=device)


def sample(logits: torch.Tensor, params: torch.Tensor, tokens_out: torch.Tensor, *, seed: int = 0,
           counter: Optional[torch.Tensor] = None, uniforms_out: Optional[torch.Tensor] = None) -> None:
    """``mk_sample`` on the current stream: next tokens from fp32 logits [B, V]
    with per-row (top_k, top_p, temperature); ``counter`` [B] int32 (e.g. the
    positions) feeds the Philox counter."""
    if logits.dtype != torch.float32 or logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be fp32 [B, V] with unit column stride")
    B, V = logits.shape
    if params.shape != (B, 3) or params.dtype != torch.float32 or not params.is_contiguous():
        raise ValueError("params must be contiguous fp32 [B, 3]")
    if tokens_out.dtype != torch.int32 or tokens_out.numel() < B:
        raise ValueError("tokens_out must be int32 with at least B elements")
    a = MkSampleArgs(logits.data_ptr(), B, V, logits.stride(0), params.data_ptr(), seed & 0xFFFFFFFFFFFFFFFF,
                     _ptr(counter), tokens_out.data_ptr(), _ptr(uniforms_out), current_stream_ptr())
    rc = load().mk_sample(ctypes.byref(a))
    if rc != MK_OK:
        raise MkError(rc, load().mk_sample_last_error().decode(errors="replace"))


class StepLauncher:
    """A prebuilt ``mk_decode_step`` call: the argument struct is built once and
    every ``launch()`` enqueues the same step on the stream. With
    ``next_token`` aliasing ``tokens`` and ``MK_FLAG_ADVANCE`` the launches form
    an autoregressive loop that needs no host work between steps."""

    def __init__(self, weights: MkWeights, ws: Workspace, k_caches: Sequence[torch.Tensor],
                 v_caches: Sequence[torch.Tensor], pos: torch.Tensor, *,
                 tokens: Optional[torch.Tensor] = None, hidden_in: Optional[torch.Tensor] = None,
                 hidden_out: Optional[torch.Tensor] = None, logits: Optional[torch.Tensor] = None,
                 next_token: Optional[torch.Tensor] = None, first_layer: int = 0,
                 n_layers: Optional[int] = None, flags: int = 0, batch: int = 1,
                 stream: Optional[torch.cuda.Stream] = None, trace: Optional[torch.Tensor] = None):
        n = len(k_caches) if n_layers is None else n_layers
        self._keep = (weights, ws, list(k_caches), list(v_caches), pos, tokens, hidden_in, hidden_out,
                      logits, next_token, trace)
        self._kc = (c_void_p * n)(*[t.data_ptr() for t in k_caches[:n]])
        self._vc = (c_void_p * n)(*[t.data_ptr() for t in v_caches[:n]])
        st = (stream or torch.cuda.current_stream()).cuda_stream
        self.args = MkStepArgs(first_layer, n, batch, int(k_caches[0].shape[-2]),
                               ctypes.cast(self._kc, POINTER(c_void_p)), ctypes.cast(self._vc, POINTER(c_void_p)),
                               _ptr(tokens), _ptr(hidden_in), _ptr(pos), _ptr(hidden_out), _ptr(logits),
                               _ptr(next_token), flags, ws.buf.data_ptr(), ws.nbytes, st, _ptr(trace))
        self.weights = weights
        self.stream_ptr = st
        self._fn = load().mk_decode_step
        self._loop_fn = load().mk_decode_loop
        self._wref = ctypes.byref(self.weights)
        self._aref = ctypes.byref(self.args)

    def launch(self) -> None:
        rc = self._fn(self._wref, self._aref)
        if rc != MK_OK:
            check(rc)

    def loop(self, n_steps: int, tokens_out: Optional[torch.Tensor] = None,
             step_clock: Optional[torch.Tensor] = None) -> None:
        """``mk_decode_loop`` with the same arguments: ``n_steps`` greedy steps
        in one launch (tokens_out: int32 [n_steps]; step_clock: int64
        [n_steps + 1]). No argument is rebuilt, so the host adds only the call
        itself to the launch."""
        rc = self._loop_fn(self._wref, self._aref, int(n_steps), _ptr(tokens_out), _ptr(step_clock))
        if rc != MK_OK:
            check(rc)


def header_functions(header: Path) -> List[str]:
    """Names of the functions declared in include/mk.h."""
    import re
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(mk_\w+)\s*\(", text, flags=re.M)
