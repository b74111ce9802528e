"""Python host binding of libgptoss_moe.so (the gfx950 GPT-OSS MoE block).

Mirrors the reference's MoE operator interface (src/model/moe_layer.cu:
1556-1615: moe_layer_create / init / forward / forward_prenormed /
get_ffn_norm_weight / destroy) and its kernel launchers, over the C ABI
declared in include/gptoss_moe.h.  Device memory is held in torch tensors
(plumbing only); every computation runs in the HIP library, and importing
this module without the built library raises immediately.

bf16 tensors are passed as torch.bfloat16 (or their int16/uint16 bit views).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
# GPTOSS_MOE_LIB: another build of the same library (the sanitizer build of
# tests/sanitize loads its instrumented copy this way)
LIB_PATH = os.environ.get("GPTOSS_MOE_LIB") or os.path.join(HERE, "libgptoss_moe.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() (make -C hip-kernels_amd)")

_lib = ctypes.CDLL(LIB_PATH)

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t

GPTOSS_OK = 0
GPTOSS_ERR_INVALID = 1
GPTOSS_ERR_UNSUPPORTED = 2
GPTOSS_ERR_HIP = 3
GPTOSS_ERR_STATE = 4
GPTOSS_ERR_OOM = 5
GPTOSS_ERR_NOT_FOUND = 6
GPTOSS_ERR_IO = 7


class GptossError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[gptoss_moe status {code}] {msg}")
        self.code = code


class ValueErrorG(GptossError, ValueError):
    """Invalid argument (status GPTOSS_ERR_INVALID); also a ValueError, as the
    reference bindings map argument errors to ValueError (bindings.cpp:105-116)."""


class MoeConfig(ctypes.Structure):
    _fields_ = [("hidden_size", _I), ("num_experts", _I), ("top_k", _I), ("intermediate_size", _I),
                ("swiglu_alpha", _F), ("swiglu_limit", _F), ("rms_norm_eps", _F), ("logits_fp32", _I),
                ("max_tokens", _I), ("prefill_min_tokens", _I), ("decode_exact", _I),
                ("prefill_block_scaled", _I)]


class MoeWeights(ctypes.Structure):
    _fields_ = [("moe_norm_weight", _P), ("router_weight", _P), ("router_bias", _P),
                ("gate_up_bias", _P), ("down_bias", _P),
                ("mlp1_packed", ctypes.POINTER(_P)), ("mlp1_scales", ctypes.POINTER(_P)),
                ("mlp2_packed", ctypes.POINTER(_P)), ("mlp2_scales", ctypes.POINTER(_P)),
                ("mlp1_tiled_nibbles", _P), ("mlp1_tiled_scales", _P),
                ("mlp2_tiled_nibbles", _P), ("mlp2_tiled_scales", _P)]


class MoeTrace(ctypes.Structure):
    _fields_ = [("logits", _P), ("expert_indices", _P), ("expert_weights", _P), ("expert_counts", _P),
                ("expert_offsets", _P), ("gather_map", _P), ("perm_token", _P), ("active_experts", _P),
                ("n_active", _P), ("gate_up", _P), ("act", _P), ("expert_out", _P)]


class TensorInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_char_p), ("ndim", _I),
                ("shape", ctypes.c_int64 * 8), ("nbytes", ctypes.c_uint64), ("data", _P), ("shard", _I)]


class ProfRecord(ctypes.Structure):
    _fields_ = [("host_us", ctypes.c_double), ("num_tokens", _I), ("prefill", _I),
                ("start_ms", _F * 4), ("dur_ms", _F * 4)]


def _sig(name, args, res=_I):
    f = getattr(_lib, name)
    f.argtypes = args
    f.restype = res
    return f


_sig("gptoss_last_error", [], ctypes.c_char_p)
_sig("gptoss_abi_version", [])
_sig("gptoss_moe_config_default", [ctypes.POINTER(MoeConfig), _I, _I])
_sig("gptoss_mxfp4_tiled_size", [_I, _I, ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)])
_sig("gptoss_mxfp4_pack_tiled", [_P, _P, _I, _I, _P, _P, _P])
_sig("gptoss_moe_layer_create", [], _P)
_sig("gptoss_moe_layer_init", [_P, ctypes.POINTER(MoeConfig), _I, ctypes.POINTER(MoeWeights)])
_sig("gptoss_moe_layer_workspace_bytes", [ctypes.POINTER(MoeConfig)], _SZ)
_sig("gptoss_moe_layer_init_with_workspace", [_P, ctypes.POINTER(MoeConfig), _I, ctypes.POINTER(MoeWeights), _P,
                                               _SZ])
_sig("gptoss_moe_layer_forward", [_P, _P, _P, _I, _P])
_sig("gptoss_moe_layer_forward_prenormed", [_P, _P, _P, _P, _I, _P])
_sig("gptoss_moe_layer_forward_residual", [_P, _P, _P, _P, _P, _I, _P])
_sig("gptoss_moe_layer_forward_routed", [_P, _P, _P, _P, _P, _P, _I, _P])
_sig("gptoss_moe_layer_forward_prenormed_noalloc", [_P, _P, _P, _P, _I, _P])
_sig("gptoss_moe_layer_get_ffn_norm_weight", [_P], _P)
_sig("gptoss_moe_layer_destroy", [_P], None)
_sig("gptoss_moe_layer_init_from_checkpoint", [_P, ctypes.POINTER(MoeConfig), _I, _P, _I])
_sig("gptoss_checkpoint_open", [ctypes.c_char_p, ctypes.POINTER(_P)])
_sig("gptoss_checkpoint_close", [_P], None)
_sig("gptoss_checkpoint_num_tensors", [_P])
_sig("gptoss_checkpoint_tensor_at", [_P, _I, ctypes.POINTER(TensorInfo)])
_sig("gptoss_checkpoint_find", [_P, ctypes.c_char_p, ctypes.POINTER(TensorInfo)])
_sig("gptoss_checkpoint_set_staging_bytes", [_P, _SZ])
_sig("gptoss_moe_layer_get_config", [_P, ctypes.POINTER(MoeConfig), ctypes.POINTER(_I)])
_HOOK = ctypes.CFUNCTYPE(None, _P, _I, _P, _P, _I, _P)
_sig("gptoss_moe_stack_create", [ctypes.POINTER(MoeConfig), _I, _P, _I, _I, ctypes.POINTER(_P)])
_sig("gptoss_moe_stack_create_from_layers", [ctypes.POINTER(_P), _I, ctypes.POINTER(_P)])
_sig("gptoss_moe_stack_io", [_P, ctypes.POINTER(_P), ctypes.POINTER(_P), ctypes.POINTER(_I), ctypes.POINTER(_I)])
_sig("gptoss_moe_stack_bind", [_P, _P, _P])
_sig("gptoss_moe_stack_layer", [_P, _I, ctypes.POINTER(_P)])
_sig("gptoss_moe_stack_decode_step", [_P, _I, _HOOK, _P, _I, _P])
_sig("gptoss_moe_stack_destroy", [_P], None)
_sig("gptoss_moe_layer_trace", [_P, ctypes.POINTER(MoeTrace)])
_sig("gptoss_moe_layer_set_trace_gate_up", [_P, _I])
_sig("gptoss_moe_layer_set_profiling", [_P, _I])
_sig("gptoss_moe_layer_profile_read", [_P, ctypes.POINTER(_F), ctypes.POINTER(_F), ctypes.POINTER(_F),
                                        ctypes.POINTER(_F), ctypes.POINTER(_I)])
_sig("gptoss_moe_layer_profile_records", [_P, ctypes.POINTER(ProfRecord), _I, ctypes.POINTER(_I)])
_sig("gptoss_moe_route_scratch_bytes", [_I, _I, _I], _SZ)
_sig("gptoss_moe_route", [_P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P])
_sig("gptoss_topk_softmax_forward", [_P, _I, _P, _P, _P, _I, _I, _I, _P])
_sig("gptoss_moe_permute_plan", [_P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P])
_sig("gptoss_moe_scatter_tokens", [_P, _P, _P, _I, _I, _I, _P])
_sig("gptoss_mxfp4_gemv_forward", [_P, _I, _P, _P, _P, _P, _I, _I, _P])
_sig("gptoss_swiglu_forward", [_P, _P, _I, _I, _F, _F, _P])
_sig("gptoss_fused_residual_rmsnorm_forward", [_P, _P, _P, _P, _P, _I, _I, _F, _P])
_sig("gptoss_moe_combine_forward", [_P, _P, _P, _P, _P, _I, _I, _I, _P])
_sig("gptoss_mxfp4_dequant", [_P, _P, _I, _I, _P, _P])
_sig("gptoss_moe_grouped_mxfp4_gemm", [_P, _P, _P, _I, _I, _P, _P, _P, _I, _I, _I, _F, _F, _P, _P, _P])

lib = _lib


def check(rc: int) -> None:
    if rc != GPTOSS_OK:
        msg = _lib.gptoss_last_error().decode()
        if rc == GPTOSS_ERR_INVALID:
            raise ValueErrorG(rc, msg)
        raise GptossError(rc, msg)


def _ptr(t):
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _bad(msg: str):
    raise ValueErrorG(GPTOSS_ERR_INVALID, msg)


def _check_tensor(name: str, t, device: int, dtype_size: int, cols: int, rows: int | None = None,
                  dtypes=None) -> None:
    """A contiguous 2-D tensor on cuda:`device` with `cols` columns (and
    `rows` rows when given) of `dtype_size`-byte elements; dtypes, when given,
    is the set of accepted torch dtypes.  The kernels read and write raw rows
    of that shape, so anything else is refused before the library sees it."""
    if not isinstance(t, torch.Tensor):
        _bad(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.dim() != 2:
        _bad(f"{name} must be 2-D, got shape {tuple(t.shape)}")
    if t.shape[1] != cols or (rows is not None and t.shape[0] != rows):
        want = f"[{rows if rows is not None else 'T'}, {cols}]"
        _bad(f"{name} has shape {tuple(t.shape)}, expected {want}")
    if dtypes is not None and t.dtype not in dtypes:
        _bad(f"{name} has dtype {t.dtype}, expected one of {sorted(str(d) for d in dtypes)}")
    if t.element_size() != dtype_size:
        _bad(f"{name} has {t.element_size()}-byte elements, expected {dtype_size}")
    if not t.is_contiguous():
        _bad(f"{name} must be contiguous")
    if t.device.type != "cuda" or t.device.index != device:
        _bad(f"{name} is on {t.device}, the layer is on cuda:{device}")


_BF16 = (torch.bfloat16, torch.int16, torch.uint16)


def _stream(stream):
    if stream is None:
        return torch.cuda.current_stream().cuda_stream if torch.cuda.is_available() else None
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def default_config(num_experts: int = 128, max_tokens: int = 64, logits_fp32: bool = False,
                   prefill_min_tokens: int | None = None, decode_exact: bool = False,
                   prefill_block_scaled: int | None = None) -> MoeConfig:
    cfg = MoeConfig()
    check(_lib.gptoss_moe_config_default(ctypes.byref(cfg), num_experts, max_tokens))
    cfg.logits_fp32 = 1 if logits_fp32 else 0
    if prefill_min_tokens is not None:
        cfg.prefill_min_tokens = prefill_min_tokens
    cfg.decode_exact = 1 if decode_exact else 0
    if prefill_block_scaled is not None:
        cfg.prefill_block_scaled = int(prefill_block_scaled)
    return cfg


def workspace_bytes(cfg: MoeConfig) -> int:
    """Bytes of forward scratch a layer of this config needs (0: invalid config)."""
    return _lib.gptoss_moe_layer_workspace_bytes(ctypes.byref(cfg))


def tiled_size(N: int, K: int):
    nb = _SZ()
    sb = _SZ()
    check(_lib.gptoss_mxfp4_tiled_size(N, K, ctypes.byref(nb), ctypes.byref(sb)))
    return nb.value, sb.value


def pack_tiled(packed: torch.Tensor, scales: torch.Tensor, N: int, K: int, out_nib=None, out_sc=None, stream=None):
    """Reference-layout MXFP4 [N][K/2] + [N][K/32] (uint8, device) -> tiled layout."""
    nb, sb = tiled_size(N, K)
    if out_nib is None:
        out_nib = torch.empty(nb, dtype=torch.uint8, device=packed.device)
    if out_sc is None:
        out_sc = torch.empty(sb, dtype=torch.uint8, device=packed.device)
    check(_lib.gptoss_mxfp4_pack_tiled(_ptr(packed), _ptr(scales), N, K, _ptr(out_nib), _ptr(out_sc),
                                       _stream(stream)))
    return out_nib, out_sc


@dataclass
class Trace:
    logits: int
    expert_indices: int
    expert_weights: int
    expert_counts: int
    expert_offsets: int
    gather_map: int
    perm_token: int
    active_experts: int
    n_active: int
    gate_up: int
    act: int
    expert_out: int


class MoELayer:
    """gptoss::MoELayer replacement (moe_layer.cu:607-1549) on one GPU.

    init() takes either the reference per-expert MXFP4 tables (lists of device
    tensors, packed and tiled by the library) or pre-tiled expert-major
    buffers (borrowed).  Tensors passed to init() must outlive the layer."""

    def __init__(self):
        self._h = _lib.gptoss_moe_layer_create()
        if not self._h:
            raise GptossError(GPTOSS_ERR_OOM, "gptoss_moe_layer_create failed")
        self._keep = []
        self._owned = True
        self.cfg = None
        self.device = None

    @classmethod
    def _borrow(cls, handle: int) -> "MoELayer":
        """A view of a layer owned elsewhere (a stack's); destroy() is a no-op."""
        self = cls.__new__(cls)
        self._h, self._keep, self._owned = handle, [], False
        self.cfg = MoeConfig()
        dev = _I()
        check(_lib.gptoss_moe_layer_get_config(handle, ctypes.byref(self.cfg), ctypes.byref(dev)))
        self.device = dev.value
        return self

    def init(self, cfg: MoeConfig, device_id: int, router_weight, router_bias=None, gate_up_bias=None,
             down_bias=None, moe_norm_weight=None, mlp1=None, mlp2=None, tiled=None,
             workspace=None) -> "MoELayer":
        """mlp1/mlp2: (list of packed tensors, list of scale tensors) per expert.
        tiled: (w1_nibbles, w1_scales, w2_nibbles, w2_scales) expert-major buffers.
        workspace: a device tensor of at least workspace_bytes(cfg) bytes for
        the forward scratch, shareable by layers run one after another on one
        stream (None: the layer allocates its own)."""
        wt = MoeWeights()
        wt.moe_norm_weight = _ptr(moe_norm_weight)
        wt.router_weight = _ptr(router_weight)
        wt.router_bias = _ptr(router_bias)
        wt.gate_up_bias = _ptr(gate_up_bias)
        wt.down_bias = _ptr(down_bias)
        if tiled is not None:
            wt.mlp1_tiled_nibbles, wt.mlp1_tiled_scales, wt.mlp2_tiled_nibbles, wt.mlp2_tiled_scales = (
                _ptr(t) for t in tiled)
        else:
            arrs = []
            for lst in (mlp1[0], mlp1[1], mlp2[0], mlp2[1]):
                a = (_P * len(lst))(*[_ptr(t) for t in lst])
                arrs.append(a)
            self._keep.append(arrs)
            wt.mlp1_packed = ctypes.cast(arrs[0], ctypes.POINTER(_P))
            wt.mlp1_scales = ctypes.cast(arrs[1], ctypes.POINTER(_P))
            wt.mlp2_packed = ctypes.cast(arrs[2], ctypes.POINTER(_P))
            wt.mlp2_scales = ctypes.cast(arrs[3], ctypes.POINTER(_P))
        if workspace is None:
            check(_lib.gptoss_moe_layer_init(self._h, ctypes.byref(cfg), device_id, ctypes.byref(wt)))
        else:
            nbytes = workspace.numel() * workspace.element_size()
            check(_lib.gptoss_moe_layer_init_with_workspace(self._h, ctypes.byref(cfg), device_id, ctypes.byref(wt),
                                                            _ptr(workspace), nbytes))
            self._keep.append(workspace)
        self.cfg = cfg
        self.device = device_id
        return self

    def init_from_checkpoint(self, cfg: MoeConfig, device_id: int, ckpt: "Checkpoint",
                             layer_index: int) -> "MoELayer":
        """Layer `layer_index` of a safetensors checkpoint (WeightLoader's MoE
        part, weight_loader.cu:1083-1165): the layer owns one device
        allocation with every weight, the experts already tiled."""
        check(_lib.gptoss_moe_layer_init_from_checkpoint(self._h, ctypes.byref(cfg), device_id, ckpt._h,
                                                         layer_index))
        self.cfg = cfg
        self.device = device_id
        return self

    def _rows(self, name: str, t, T: int | None = None) -> int:
        """Checks a bf16 [T, hidden_size] activation tensor on the layer's
        device; returns T."""
        if self.cfg is None:
            raise GptossError(GPTOSS_ERR_STATE, "layer not initialised")
        _check_tensor(name, t, self.device, 2, self.cfg.hidden_size, T, _BF16)
        return t.shape[0]

    def _out(self, out, like, T: int):
        if out is None:
            return torch.empty_like(like)
        self._rows("out", out, T)
        return out

    def forward(self, x, out=None, stream=None):
        """out = x + MoE(RMSNorm(x)) (moe_layer_forward)."""
        T = self._rows("x", x)
        out = self._out(out, x, T)
        check(_lib.gptoss_moe_layer_forward(self._h, _ptr(x), _ptr(out), T, _stream(stream)))
        return out

    def forward_prenormed(self, normed, residual=None, out=None, stream=None):
        """out = residual + MoE(normed) (moe_layer_forward_prenormed)."""
        T = self._rows("normed", normed)
        if residual is not None:
            self._rows("residual", residual, T)
        out = self._out(out, normed, T)
        check(_lib.gptoss_moe_layer_forward_prenormed(self._h, _ptr(normed), _ptr(residual), _ptr(out), T,
                                                      _stream(stream)))
        return out

    def forward_prenormed_noalloc(self, normed, residual=None, out=None, stream=None):
        """forward_prenormed with the forward scratch in the library's static
        device array (no allocation; up to 64 tokens; calls overlapping on one
        GPU race).  `out` must be given: this call allocates nothing."""
        if out is None:
            _bad("forward_prenormed_noalloc needs an output tensor (it allocates nothing)")
        T = self._rows("normed", normed)
        if residual is not None:
            self._rows("residual", residual, T)
        self._rows("out", out, T)
        check(_lib.gptoss_moe_layer_forward_prenormed_noalloc(self._h, _ptr(normed), _ptr(residual), _ptr(out), T,
                                                              _stream(stream)))
        return out

    def forward_residual(self, residual, delta, residual_out=None, out=None, stream=None):
        """The decode step's residual add + RMSNorm + MoE in one call:
        s = residual + delta; residual_out (optional) = bf16(s);
        out = bf16(s) + MoE(RMSNorm(s)).  residual_out must not share memory
        with residual or delta.  Returns out."""
        T = self._rows("residual", residual)
        self._rows("delta", delta, T)
        if residual_out is not None:
            self._rows("residual_out", residual_out, T)
        out = self._out(out, residual, T)
        check(_lib.gptoss_moe_layer_forward_residual(self._h, _ptr(residual), _ptr(delta), _ptr(residual_out),
                                                     _ptr(out), T, _stream(stream)))
        return out

    def forward_routed(self, normed, expert_indices, expert_weights, residual=None, out=None, stream=None):
        """out = residual + sum_k w * FFN_idx(normed) with the routing given
        (int32 [T][k] indices, fp32 [T][k] weights, on the device)."""
        T = self._rows("normed", normed)
        if residual is not None:
            self._rows("residual", residual, T)
        k = self.cfg.top_k
        _check_tensor("expert_indices", expert_indices, self.device, 4, k, T, (torch.int32,))
        _check_tensor("expert_weights", expert_weights, self.device, 4, k, T, (torch.float32,))
        out = self._out(out, normed, T)
        check(_lib.gptoss_moe_layer_forward_routed(self._h, _ptr(normed), _ptr(residual), _ptr(expert_indices),
                                                   _ptr(expert_weights), _ptr(out), T, _stream(stream)))
        return out

    def get_ffn_norm_weight(self) -> int:
        return _lib.gptoss_moe_layer_get_ffn_norm_weight(self._h) or 0

    def set_trace_gate_up(self, enable: bool) -> None:
        check(_lib.gptoss_moe_layer_set_trace_gate_up(self._h, 1 if enable else 0))

    def set_profiling(self, max_forwards: int) -> None:
        check(_lib.gptoss_moe_layer_set_profiling(self._h, max_forwards))

    def profile_read(self):
        """(route_ms, w1_ms, w2_ms, combine_ms, n_forwards) summed over the
        recorded forwards (route_ms is the plan launch for forward_routed)."""
        r, a, b, c, n = _F(), _F(), _F(), _F(), _I()
        check(_lib.gptoss_moe_layer_profile_read(self._h, ctypes.byref(r), ctypes.byref(a), ctypes.byref(b),
                                                 ctypes.byref(c), ctypes.byref(n)))
        return r.value, a.value, b.value, c.value, n.value

    def profile_records(self):
        """Per recorded forward: dict(host_us, num_tokens, prefill, start_ms[4],
        dur_ms[4]) for the route (or plan), gate_up, down and combine launches."""
        n = _I()
        check(_lib.gptoss_moe_layer_profile_records(self._h, None, 0, ctypes.byref(n)))
        recs = (ProfRecord * max(n.value, 1))()
        check(_lib.gptoss_moe_layer_profile_records(self._h, recs, n.value, ctypes.byref(n)))
        return [dict(host_us=r.host_us, num_tokens=r.num_tokens, prefill=r.prefill,
                     start_ms=list(r.start_ms), dur_ms=list(r.dur_ms)) for r in recs[:n.value]]

    def trace(self) -> Trace:
        t = MoeTrace()
        check(_lib.gptoss_moe_layer_trace(self._h, ctypes.byref(t)))
        return Trace(*[getattr(t, f[0]) or 0 for f in MoeTrace._fields_])

    def destroy(self) -> None:
        if self._h:
            if self._owned:
                _lib.gptoss_moe_layer_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Checkpoint:
    """A safetensors checkpoint (a directory of shards or one file), mapped
    read-only: WeightLoader's shard scan, header parse and name index
    (weight_loader.cu:297-345, 456-575).  Host-only: opening and reading
    tensors needs no GPU."""

    _NP = {"BF16": "<u2", "F16": "<f2", "F32": "<f4", "F64": "<f8", "U8": "u1", "I8": "i1", "BOOL": "u1",
           "I16": "<i2", "U16": "<u2", "I32": "<i4", "U32": "<u4", "I64": "<i8", "U64": "<u8"}

    def __init__(self, path: str):
        h = _P()
        check(_lib.gptoss_checkpoint_open(os.fsencode(path), ctypes.byref(h)))
        self._h = h.value

    def __len__(self) -> int:
        return _lib.gptoss_checkpoint_num_tensors(self._h)

    @staticmethod
    def _info(ti: TensorInfo) -> dict:
        return {"name": ti.name.decode(), "dtype": ti.dtype.decode(), "shape": tuple(ti.shape[:ti.ndim]),
                "nbytes": ti.nbytes, "data": ti.data or 0, "shard": ti.shard}

    def names(self):
        out = []
        ti = TensorInfo()
        for i in range(len(self)):
            check(_lib.gptoss_checkpoint_tensor_at(self._h, i, ctypes.byref(ti)))
            out.append(ti.name.decode())
        return out

    def info(self, name: str):
        """dict(name, dtype, shape, nbytes, data, shard), or None when absent."""
        ti = TensorInfo()
        rc = _lib.gptoss_checkpoint_find(self._h, name.encode(), ctypes.byref(ti))
        if rc == GPTOSS_ERR_NOT_FOUND:
            return None
        check(rc)
        return self._info(ti)

    def numpy(self, name: str):
        """A copy of the tensor as a numpy array (bf16 as uint16; dtypes
        outside the safetensors list as flat bytes)."""
        import numpy as np
        inf = self.info(name)
        if inf is None:
            raise KeyError(name)
        raw = ctypes.string_at(inf["data"], inf["nbytes"]) if inf["nbytes"] else b""
        dt = self._NP.get(inf["dtype"])
        a = np.frombuffer(raw, dtype=dt or "u1")
        return (a.reshape(inf["shape"]) if dt else a).copy()

    def _router_weight(self, layer: int):
        for n in ("mlp.gate.weight", "mlp.router.weight"):
            inf = self.info(f"model.layers.{layer}.{n}")
            if inf is not None:
                return inf
        return None

    def num_moe_layers(self) -> int:
        """Layers 0, 1, ... that have a router weight."""
        n = 0
        while self._router_weight(n) is not None:
            n += 1
        return n

    def moe_shape(self, layer: int = 0):
        """(E, H, I) of a layer, from its router weight [E][H] and its gate_up
        blocks or biases ([E][2I]...)."""
        rw = self._router_weight(layer)
        if rw is None:
            raise GptossError(GPTOSS_ERR_NOT_FOUND, f"no router weight for layer {layer}")
        E, H = rw["shape"]
        P = f"model.layers.{layer}.mlp.experts."
        for n in ("gate_up_proj_blocks", "gate_up_proj_bias", "0.mlp1.weight", "0.gate_up_proj.weight",
                  "0.w1.weight"):
            inf = self.info(P + n)
            if inf is not None:
                return E, H, inf["shape"][1 if n.startswith("gate_up") else 0] // 2
        raise GptossError(GPTOSS_ERR_NOT_FOUND, f"no gate_up tensor for layer {layer}")

    def set_staging_bytes(self, nbytes: int) -> None:
        check(_lib.gptoss_checkpoint_set_staging_bytes(self._h, nbytes))

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.gptoss_checkpoint_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class MoEStack:
    """The MoE half of the engine's decode step over a stack of layers
    (transformer.cu:653-753): per layer, an optional hook writes the layer's
    delta from the current residual (the engine's attention), then
    residual = bf16(residual + delta) + MoE(RMSNorm(residual + delta)),
    in place.  decode_step(use_graph=True) replays one hipGraph per token
    count, captured on first use.  The residual and deltas live in torch
    tensors bound to the stack: `residual` [max_tokens][H] and `deltas`
    [num_layers][max_tokens][H], bf16."""

    def __init__(self, handle: int, layers=None):
        self._h = handle
        self._layers = layers  # layers borrowed by the stack, kept alive here
        self._hooks = {}
        r, d, mt, nl = _P(), _P(), _I(), _I()
        check(_lib.gptoss_moe_stack_io(self._h, ctypes.byref(r), ctypes.byref(d), ctypes.byref(mt), ctypes.byref(nl)))
        self.max_tokens, self.num_layers = mt.value, nl.value
        L0 = _P()
        check(_lib.gptoss_moe_stack_layer(self._h, 0, ctypes.byref(L0)))
        cfg, dev = MoeConfig(), _I()
        check(_lib.gptoss_moe_layer_get_config(L0.value, ctypes.byref(cfg), ctypes.byref(dev)))
        self.cfg, self.device = cfg, dev.value
        H = cfg.hidden_size
        device = torch.device("cuda", self.device)
        self.residual = torch.zeros((self.max_tokens, H), dtype=torch.bfloat16, device=device)
        self.deltas = torch.zeros((self.num_layers, self.max_tokens, H), dtype=torch.bfloat16, device=device)
        check(_lib.gptoss_moe_stack_bind(self._h, _ptr(self.residual), _ptr(self.deltas)))

    @classmethod
    def from_checkpoint(cls, cfg: MoeConfig, device_id: int, ckpt: "Checkpoint", first_layer: int = 0,
                        num_layers: int | None = None) -> "MoEStack":
        if num_layers is None:
            num_layers = ckpt.num_moe_layers() - first_layer
        h = _P()
        check(_lib.gptoss_moe_stack_create(ctypes.byref(cfg), device_id, ckpt._h, first_layer, num_layers,
                                           ctypes.byref(h)))
        return cls(h.value)

    @classmethod
    def from_layers(cls, layers) -> "MoEStack":
        arr = (_P * len(layers))(*[L._h for L in layers])
        h = _P()
        check(_lib.gptoss_moe_stack_create_from_layers(arr, len(layers), ctypes.byref(h)))
        return cls(h.value, layers=list(layers))

    def layer(self, i: int) -> MoELayer:
        h = _P()
        check(_lib.gptoss_moe_stack_layer(self._h, i, ctypes.byref(h)))
        return MoELayer._borrow(h.value)

    def _c_hook(self, hook):
        """One C function pointer per Python hook, so that the same hook
        finds its captured graph again."""
        if hook is None:
            return _HOOK()
        key = id(hook)
        if key not in self._hooks:
            def tramp(_user, layer, residual, delta, T, stream, _hook=hook):
                _hook(layer, residual or 0, delta or 0, T, stream or 0)
            self._hooks[key] = (hook, _HOOK(tramp))
        return self._hooks[key][1]

    def decode_step(self, T: int, hook=None, use_graph: bool = True, stream=None) -> torch.Tensor:
        """One step on residual[:T] with deltas[:, :T].  hook(layer,
        residual_ptr, delta_ptr, T, stream_ptr) runs before each layer (only
        while a graph is captured when use_graph).  Returns residual[:T]."""
        check(_lib.gptoss_moe_stack_decode_step(self._h, T, self._c_hook(hook), None, 1 if use_graph else 0,
                                                _stream(stream)))
        return self.residual[:T]

    def destroy(self) -> None:
        if getattr(self, "_h", None):
            _lib.gptoss_moe_stack_destroy(self._h)
            self._h = None
        self._layers = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class ModelConfig:
    """The MoE constants of GPT-OSS-120B, as the reference's read-only
    gptoss.ModelConfig exposes them (bindings.cpp:317-400, config.h)."""
    num_layers = 36
    hidden_size = 2880
    num_experts = 128
    num_active_experts = 4
    expert_intermediate_size = 2880
    rms_norm_eps = 1e-5
    swiglu_alpha = 1.702
    swiglu_limit = 7.0


class MoEEngine:
    """The InferenceEngine lifecycle (bindings.cpp:221-311: init(weights_dir),
    shutdown(), is_initialized) over the MoE half of the model: init() loads
    every MoE layer of a safetensors checkpoint into one stack on one GPU;
    decode_step() runs the per-layer residual add + RMSNorm + MoE of the
    decode step for all layers, as one cached hipGraph per batch size.  The
    attention that produces each layer's delta is the caller's (a hook, or
    deltas written beforehand)."""

    def __init__(self):
        self._stack = None

    def init(self, weights_dir: str, max_tokens: int = 64, device_id: int = 0, num_layers: int | None = None,
             top_k: int = ModelConfig.num_active_experts) -> "MoEEngine":
        if self._stack is not None:
            raise GptossError(GPTOSS_ERR_STATE, "[MoEEngine] Already initialized")
        with Checkpoint(weights_dir) as ck:
            E, H, I = ck.moe_shape(0)
            cfg = default_config(E, max_tokens)
            cfg.hidden_size, cfg.intermediate_size, cfg.top_k = H, I, top_k
            self._stack = MoEStack.from_checkpoint(cfg, device_id, ck, 0, num_layers)
        return self

    @property
    def is_initialized(self) -> bool:
        return self._stack is not None

    @property
    def stack(self) -> MoEStack:
        if self._stack is None:
            raise GptossError(GPTOSS_ERR_STATE, "[MoEEngine] Not initialized")
        return self._stack

    def decode_step(self, hidden: torch.Tensor, deltas: torch.Tensor | None = None, hook=None,
                    use_graph: bool = True) -> torch.Tensor:
        """hidden [T][H] bf16 (the residual stream entering layer 0); deltas
        [num_layers][T][H] (or a hook).  Returns the residual after the last
        layer, [T][H]."""
        st = self.stack
        T = hidden.shape[0]
        st.residual[:T].copy_(hidden)
        if deltas is not None:
            st.deltas[:, :T].copy_(deltas)
        return st.decode_step(T, hook=hook, use_graph=use_graph).clone()

    def shutdown(self) -> None:
        if self._stack is not None:
            self._stack.destroy()
            self._stack = None

    def __repr__(self) -> str:
        n = self._stack.num_layers if self._stack is not None else 0
        return f"<gptoss_moe.MoEEngine initialized={self.is_initialized} layers={n}>"


# ---------------------------------------------------------------------------
# device buffer readback (for traces, which are raw device pointers)
# ---------------------------------------------------------------------------
_hip = None


def copy_device_to_tensor(ptr: int, nbytes: int, dtype=torch.uint8, device="cuda") -> torch.Tensor:
    """Copy `nbytes` at device pointer `ptr` into a new device tensor (hipMemcpy D2D)."""
    global _hip
    if _hip is None:
        # same SONAME as the runtime torch loaded, so this binds to that instance
        _hip = ctypes.CDLL("libamdhip64.so.7")
        _hip.hipMemcpy.argtypes = [_P, _P, _SZ, _I]
        _hip.hipMemcpy.restype = _I
    out = torch.empty(nbytes, dtype=torch.uint8, device=device)
    if nbytes:
        rc = _hip.hipMemcpy(out.data_ptr(), ptr, nbytes, 3)  # hipMemcpyDeviceToDevice
        if rc != 0:
            raise GptossError(GPTOSS_ERR_HIP, f"hipMemcpy failed ({rc})")
    return out.view(dtype)


# ---------------------------------------------------------------------------
# stage entry points
# ---------------------------------------------------------------------------
def route_scratch(T: int, E: int, top_k: int, device="cuda") -> torch.Tensor:
    """Zero-filled scratch for route() (the call leaves its counters zero)."""
    return torch.zeros(_lib.gptoss_moe_route_scratch_bytes(T, E, top_k), dtype=torch.uint8, device=device)


def route(x, router_w, router_b, top_k: int, logits_fp32: bool = False, stream=None, out=None, scratch=None):
    """Router GEMV + top-k softmax (gptoss_moe_route): (logits, idx, weights).
    out: preallocated (logits, idx, weights); scratch: from route_scratch()."""
    T, H = x.shape
    E = router_w.shape[0]
    dev = x.device
    if out is None:
        logits = torch.empty((T, E), dtype=torch.float32 if logits_fp32 else torch.bfloat16, device=dev)
        idx = torch.empty((T, top_k), dtype=torch.int32, device=dev)
        w = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    else:
        logits, idx, w = out
    if scratch is None:
        scratch = route_scratch(T, E, top_k, dev)
    check(_lib.gptoss_moe_route(_ptr(x), _ptr(router_w), _ptr(router_b), T, E, H, top_k, 1 if logits_fp32 else 0,
                                _ptr(logits), _ptr(idx), _ptr(w), _ptr(scratch), _stream(stream)))
    return logits, idx, w


def topk_softmax(logits, top_k: int, tokens_per_expert=None, stream=None):
    T, E = logits.shape
    idx = torch.empty((T, top_k), dtype=torch.int32, device=logits.device)
    w = torch.empty((T, top_k), dtype=torch.float32, device=logits.device)
    check(_lib.gptoss_topk_softmax_forward(_ptr(logits), 1 if logits.dtype == torch.float32 else 0, _ptr(idx),
                                           _ptr(w), _ptr(tokens_per_expert), T, E, top_k, _stream(stream)))
    return idx, w


def permute_plan(idx, num_experts: int, stream=None):
    T, k = idx.shape
    dev = idx.device
    S = T * k
    counts = torch.empty(num_experts, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    gmap = torch.empty(S, dtype=torch.int32, device=dev)
    ptok = torch.full((S,), -1, dtype=torch.int32, device=dev)
    active = torch.full((num_experts,), -1, dtype=torch.int32, device=dev)
    n_active = torch.empty(1, dtype=torch.int32, device=dev)
    check(_lib.gptoss_moe_permute_plan(_ptr(idx), T, k, num_experts, _ptr(counts), _ptr(offsets), _ptr(gmap),
                                       _ptr(ptok), _ptr(active), _ptr(n_active), _stream(stream)))
    return dict(counts=counts, offsets=offsets, gather_map=gmap, perm_token=ptok, active=active, n_active=n_active)


def scatter_tokens(x, gather_map, top_k: int, stream=None):
    T, H = x.shape
    out = torch.zeros((T * top_k, H), dtype=x.dtype, device=x.device)
    check(_lib.gptoss_moe_scatter_tokens(_ptr(x), _ptr(gather_map), _ptr(out), T, H, top_k, _stream(stream)))
    return out


def mxfp4_gemv(x, tiled_nib, tiled_sc, bias, N: int, K: int, stream=None):
    M = x.shape[0]
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    check(_lib.gptoss_mxfp4_gemv_forward(_ptr(x), M, _ptr(tiled_nib), _ptr(tiled_sc), _ptr(bias), _ptr(y), N, K,
                                         _stream(stream)))
    return y


def swiglu(gate_up, alpha: float = 1.702, limit: float = 7.0, stream=None):
    T, N2 = gate_up.shape
    out = torch.empty((T, N2 // 2), dtype=gate_up.dtype, device=gate_up.device)
    check(_lib.gptoss_swiglu_forward(_ptr(gate_up), _ptr(out), T, N2 // 2, alpha, limit, _stream(stream)))
    return out


def fused_residual_rmsnorm(residual, delta, weight, eps: float = 1e-5, normed=None, sum_out=None, stream=None):
    """fused_residual_rmsnorm_forward: returns (normed, sum_out)."""
    T, H = residual.shape
    if normed is None:
        normed = torch.empty_like(residual)
    if sum_out is None:
        sum_out = torch.empty_like(residual)
    check(_lib.gptoss_fused_residual_rmsnorm_forward(_ptr(residual), _ptr(delta), _ptr(weight), _ptr(normed),
                                                     _ptr(sum_out), T, H, eps, _stream(stream)))
    return normed, sum_out


def combine(expert_out, gather_map, weights, residual, T: int, H: int, top_k: int, stream=None):
    out = torch.empty((T, H), dtype=torch.bfloat16, device=expert_out.device)
    check(_lib.gptoss_moe_combine_forward(_ptr(out), _ptr(expert_out), _ptr(gather_map), _ptr(weights),
                                          _ptr(residual), T, H, top_k, _stream(stream)))
    return out


def dequant(tiled_nib, tiled_sc, N: int, K: int, stream=None):
    out = torch.empty((N, K), dtype=torch.bfloat16, device=tiled_nib.device)
    check(_lib.gptoss_mxfp4_dequant(_ptr(tiled_nib), _ptr(tiled_sc), N, K, _ptr(out), _stream(stream)))
    return out


def grouped_mxfp4_gemm(x, offsets, tiled_nib, tiled_sc, N: int, K: int, rows: int, bias=None, row_index=None,
                       swiglu: bool = False, alpha: float = 1.702, limit: float = 7.0, gate_up=None, out=None,
                       stream=None):
    """Grouped expert product on the matrix cores: rows p of expert e (offsets,
    int32 [E+1] on the device) times W_e (expert-major tiled buffers); x rows
    gathered through row_index when given.  swiglu: out is [rows][N/2]."""
    E = offsets.numel() - 1
    if out is None:
        out = torch.empty((rows, N // 2 if swiglu else N), dtype=torch.bfloat16, device=x.device)
    check(_lib.gptoss_moe_grouped_mxfp4_gemm(_ptr(x), _ptr(row_index), _ptr(offsets), E, rows, _ptr(tiled_nib),
                                             _ptr(tiled_sc), _ptr(bias), N, K, 1 if swiglu else 0, alpha, limit,
                                             _ptr(out), _ptr(gate_up), _stream(stream)))
    return out
