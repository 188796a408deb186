"""Verify-linear drop-in modules (mirrors dflash_mlx/verify_linear.py).

``QuantizedLinear`` is this framework's counterpart of ``mlx.nn.QuantizedLinear``
(same fields: ``weight`` packed words ``[N, K*bits/32]``, ``scales``,
``biases``, optional ``bias``, ``group_size``, ``bits``, ``mode``).
``VerifyQuantizedLinear`` precomputes its route once per module
(``_build_dispatch``, reference 118-309) and sends M=16 / M=4 calls to the
verify kernels; every other M goes to the stock quantized matmul.
``install_verify_linears`` swaps eligible leaves in a module tree (338-361).
"""

from __future__ import annotations

import math
from typing import Callable, Optional

import torch
from torch import nn

from . import _lib, _runtime
from .internal_debug import (
    verify_include as _debug_verify_include,
    verify_max_n as _debug_verify_max_n,
    verify_qmm_enabled as _debug_verify_qmm_enabled,
)
from .quantize import quantize
from .verify_qmm import (
    _kparts_tuning,
    _m4_ksplit_np_shape,
    qmm_multi_launch,
    _resolve_m16_ktmpl_variant,
    qmm_launch,
    quantized_matmul,
    verify_matmul,
)

_VERIFY_MAX_N_DEFAULT = 100_000

_PROJ_TAGS = {
    "mlp.gate_proj": "mlp_gate",
    "mlp.up_proj": "mlp_up",
    "mlp.down_proj": "mlp_down",
    "self_attn.q_proj": "attn_q",
    "self_attn.k_proj": "attn_k",
    "self_attn.v_proj": "attn_v",
    "self_attn.o_proj": "attn_o",
    "linear_attn.in_proj_qkv": "gdn_qkv",
    "linear_attn.in_proj_z": "gdn_z",
    "linear_attn.out_proj": "gdn_o",
}


def _path_tag(path: str) -> str:
    """dflash_mlx/verify_linear.py:47-52."""
    for suffix, tag in _PROJ_TAGS.items():
        if path.endswith(suffix):
            return tag
    return "other"


class QuantizedLinear(nn.Module):
    """Affine group-quantized linear layer, ``y = x . dequant(W)^T (+ bias)``."""

    def __init__(self, weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                 bias: Optional[torch.Tensor] = None, *, group_size: int = 64, bits: int = 4,
                 mode: str = "affine"):
        super().__init__()
        self.group_size = int(group_size)
        self.bits = int(bits)
        self.mode = mode
        self.register_buffer("weight", weight)
        self.register_buffer("scales", scales)
        self.register_buffer("biases", biases)
        if bias is not None:
            self.register_buffer("bias", bias)
        else:
            self.bias = None

    @classmethod
    def from_linear(cls, linear: nn.Linear, group_size: int = 64, bits: int = 4,
                    dtype: Optional[torch.dtype] = None) -> "QuantizedLinear":
        w_q, s, b = quantize(linear.weight.detach(), group_size, bits, dtype)
        bias = linear.bias.detach().to(s.dtype) if linear.bias is not None else None
        return cls(w_q, s, b, bias, group_size=group_size, bits=bits)

    @property
    def in_features(self) -> int:
        return int(self.weight.shape[1]) * (32 // self.bits)

    @property
    def out_features(self) -> int:
        return int(self.weight.shape[0])

    def has_bias(self) -> bool:
        return getattr(self, "bias", None) is not None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = quantized_matmul(x, self.weight, self.scales, self.biases, transpose=True,
                             group_size=self.group_size, bits=self.bits, mode=self.mode)
        return y + self.bias if self.has_bias() else y


def is_verify_eligible(ql: nn.Module, path: str = "") -> bool:
    """dflash_mlx/verify_linear.py:54-87."""
    if not isinstance(ql, QuantizedLinear):
        return False
    if getattr(ql, "bits", None) not in (4, 8):
        return False
    if getattr(ql, "group_size", None) not in (32, 64, 128):
        return False
    if getattr(ql, "mode", "affine") != "affine":
        return False
    w = ql.weight
    N = int(w.shape[0])
    K = int(w.shape[1]) * (32 // ql.bits)
    if K % 32 != 0:
        return False
    if ql.bits == 4:
        if N % 4 != 0:
            return False
    elif N % 32 != 0:
        return False
    if N >= _debug_verify_max_n(_VERIFY_MAX_N_DEFAULT):
        return False
    include = _debug_verify_include()
    if include not in ("", "all"):
        tag = _path_tag(path)
        allowed = {s.strip() for s in include.split(",") if s.strip()}
        if "mlp" in allowed:
            allowed.update({"mlp_gate", "mlp_up", "mlp_down"})
        if "attn" in allowed:
            allowed.update({"attn_q", "attn_k", "attn_v", "attn_o"})
        if "gdn" in allowed:
            allowed.update({"gdn_qkv", "gdn_z", "gdn_o"})
        if tag not in allowed:
            return False
    return True


class VerifyQuantizedLinear(QuantizedLinear):
    """``QuantizedLinear`` whose M=16 / M=4 calls take the verify kernels
    (dflash_mlx/verify_linear.py:89-116)."""

    @classmethod
    def from_quantized(cls, ql: QuantizedLinear, *,
                       enable_qmm: Optional[bool] = None) -> "VerifyQuantizedLinear":
        obj = cls(ql.weight, ql.scales, ql.biases, getattr(ql, "bias", None),
                  group_size=ql.group_size, bits=ql.bits, mode=getattr(ql, "mode", "affine"))
        object.__setattr__(obj, "_call_fn", _build_dispatch(obj, enable_qmm=enable_qmm))
        obj.requires_grad_(False)
        return obj

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._call_fn(x)


def _build_dispatch(obj: VerifyQuantizedLinear, *, enable_qmm: Optional[bool] = None):
    """dflash_mlx/verify_linear.py:118-309: route chosen once per module."""
    gs, bits, mode = obj.group_size, obj.bits, obj.mode
    N = int(obj.weight.shape[0])
    K = int(obj.weight.shape[1]) * (32 // bits)
    bias = obj.bias if obj.has_bias() else None
    qmm_enabled = _debug_verify_qmm_enabled() if enable_qmm is None else bool(enable_qmm)

    ktmpl_variant = _resolve_m16_ktmpl_variant(K, N, bits) if qmm_enabled else None
    m16_qmm = qmm_enabled and (ktmpl_variant is not None or (N % 32 == 0 and K % 32 == 0))
    m4_qmm = qmm_enabled and _m4_ksplit_np_shape(K, N, bits)
    # Reference 176-188 picks mma2big_pipe (K_PARTS 8) or mma2big for shapes
    # the K-templated kernels decline; both run the automatic plan here (the
    # K_PARTS values are Metal launch choices), or DFLASH_VERIFY_QMM_KPARTS
    # splits when the user sets it.
    m16_tuning = _kparts_tuning() if (m16_qmm and ktmpl_variant is None) else None

    def _stock(x):
        return quantized_matmul(x, obj.weight, obj.scales, obj.biases, transpose=True,
                                group_size=gs, bits=bits, mode=mode)

    if m16_qmm or m4_qmm:
        w_c = _runtime.weight_words(obj.weight)
        s_c = _runtime.aligned_contiguous(obj.scales)
        b_c = _runtime.aligned_contiguous(obj.biases)
        kernel_dtypes = (torch.bfloat16, torch.float16)
        # the (scale, bias) pair table of the streaming plans, built once per
        # module on its first GPU call (or by prewarm_verify_kernels), like
        # the reference's precomputed route; the launch plan and the result
        # do not depend on it, so a call under graph capture before it exists
        # runs without it
        pair_state = [None, obj.scales.dtype in kernel_dtypes and
                      _runtime.pair_shape(16, K, N, gs, bits)]

        def pairs_of():
            if pair_state[0] is None and pair_state[1]:
                if torch.cuda.is_current_stream_capturing():
                    return None
                pair_state[0] = _runtime.build_sb_pairs(s_c, b_c)
            return pair_state[0]

        object.__setattr__(obj, "_packed", (w_c, s_c, b_c))
        object.__setattr__(obj, "_pairs_of", pairs_of)

        def call(x: torch.Tensor) -> torch.Tensor:
            orig = x.shape
            m = math.prod(int(d) for d in orig[:-1])
            if x.dtype in kernel_dtypes and ((m == 16 and m16_qmm) or (m == 4 and m4_qmm)):
                sib = obj.__dict__.get("_sibling")
                if sib is not None:
                    y = sib[0].product(sib[1], x, m).reshape(*orig[:-1], N)
                else:
                    x2 = _runtime.aligned_contiguous(x.reshape(m, orig[-1]))
                    tuning = m16_tuning if m == 16 else None
                    y = qmm_launch(x2, w_c, s_c, b_c, N, gs, bits, tuning,
                                   pairs=pairs_of()).reshape(*orig[:-1], N)
            else:
                y = _stock(x)
            return y + bias if bias is not None else y

        return call

    def call(x: torch.Tensor) -> torch.Tensor:
        m = math.prod(int(d) for d in x.shape[:-1])
        if m == 16:
            y = verify_matmul(x, obj.weight, obj.scales, obj.biases, transpose=True,
                              group_size=gs, bits=bits)
        else:
            y = _stock(x)
        return y + bias if bias is not None else y

    return call


def _leaf_modules(model: nn.Module):
    for path, mod in model.named_modules():
        if path and not any(True for _ in mod.children()):
            yield path, mod


def _set_module(model: nn.Module, path: str, new: nn.Module) -> None:
    parent_path, _, name = path.rpartition(".")
    parent = model.get_submodule(parent_path) if parent_path else model
    if isinstance(parent, (nn.ModuleList, nn.Sequential)) and name.isdigit():
        parent[int(name)] = new
    else:
        setattr(parent, name, new)


def prewarm_verify_kernels(model: nn.Module, *, input_dtype: torch.dtype = torch.bfloat16) -> int:
    """dflash_mlx/verify_linear.py:311-336: one M=16 (and M=4 when eligible)
    call per unique (K, N, bits, group_size); also sizes this stream's
    workspace so later calls (and graph captures) do not allocate it, and
    builds every verify module's pair table."""
    seen: set[tuple] = set()
    warmed = 0
    for _, m in _leaf_modules(model):
        if not isinstance(m, VerifyQuantizedLinear):
            continue
        if "_pairs_of" in m.__dict__:
            m._pairs_of()
        K = int(m.weight.shape[1]) * (32 // m.bits)
        N = int(m.weight.shape[0])
        key = (K, N, m.bits, m.group_size)
        if key in seen:
            continue
        seen.add(key)
        dev = m.weight.device
        m(torch.zeros((1, 16, K), dtype=input_dtype, device=dev))
        warmed += 1
        if _m4_ksplit_np_shape(K, N, m.bits):
            m(torch.zeros((1, 4, K), dtype=input_dtype, device=dev))
            warmed += 1
    return warmed


# Sibling projections that read the same input in the decoder layers the
# reference targets (q/k/v of self_attn, gate/up of mlp).
_SIBLING_SETS = (("q_proj", "k_proj", "v_proj"), ("gate_proj", "up_proj"))


class SiblingGroup:
    """Verify modules of one parent that read the same input: the first member
    called with a verify-sized input computes every member's product in one
    ``dfmi_qmm_affine_multi`` launch; the others return theirs when they are
    called with the same tensor (same storage, version, shape, strides and
    stream) -- in the model's call order, with no change to the model code.
    A member called with any other input recomputes the group."""

    def __init__(self, members):
        self.members = list(members)
        self._key = None
        self._ys = None
        self._taken: set[int] = set()

    def product(self, idx: int, x: torch.Tensor, m: int) -> torch.Tensor:
        key = (x.data_ptr(), x._version, tuple(x.shape), tuple(x.stride()), x.dtype,
               _runtime.stream_ptr(x.device))
        if self._ys is not None and self._key == key and idx not in self._taken:
            y = self._ys[idx]
        else:
            x2 = _runtime.aligned_contiguous(x.reshape(m, int(x.shape[-1])))
            first = self.members[0]
            self._ys = qmm_multi_launch(x2, [(*mem._packed, mem._pairs_of())
                                             for mem in self.members],
                                        first.group_size, first.bits)
            self._key = key
            self._taken = set()
            y = self._ys[idx]
        self._taken.add(idx)
        if len(self._taken) == len(self.members):
            self._key, self._ys, self._taken = None, None, set()  # drop the references
        return y


def _group_siblings(model: nn.Module) -> int:
    """Attach a SiblingGroup to each set of sibling verify modules of one
    parent that share K, bits, group size and scale dtype and take the verify
    kernels; returns the number of groups."""
    groups = 0
    for _, parent in model.named_modules():
        for names in _SIBLING_SETS:
            mods = [getattr(parent, n, None) for n in names]
            if not all(isinstance(m, VerifyQuantizedLinear) and "_packed" in m.__dict__
                       for m in mods):
                continue
            sig = {(int(m.weight.shape[1]) * (32 // m.bits), m.bits, m.group_size, m.scales.dtype)
                   for m in mods}
            if len(sig) != 1:
                continue
            grp = SiblingGroup(mods)
            for i, m in enumerate(mods):
                object.__setattr__(m, "_sibling", (grp, i))
            groups += 1
    return groups


def install_verify_linears(model: nn.Module, *,
                           predicate: Optional[Callable[[str, QuantizedLinear], bool]] = None,
                           enable_qmm: Optional[bool] = None,
                           fuse_siblings: bool = False) -> int:
    """dflash_mlx/verify_linear.py:338-361: swap eligible QuantizedLinear
    leaves for VerifyQuantizedLinear; returns the number swapped.

    ``fuse_siblings`` (no reference counterpart, opt-in): group q/k/v and
    gate/up siblings so each set runs as one shared-activation launch
    (:class:`SiblingGroup`); every member's output equals what
    ``quantized_matmul_multi`` returns for it (plus its bias), which is
    within fp32 summation order of the member's own launch."""
    if predicate is None:
        predicate = lambda path, m: is_verify_eligible(m, path=path)  # noqa: E731
    count = 0
    for path, m in list(_leaf_modules(model)):
        if isinstance(m, VerifyQuantizedLinear):
            continue
        if isinstance(m, QuantizedLinear) and predicate(path, m):
            _set_module(model, path, VerifyQuantizedLinear.from_quantized(m, enable_qmm=enable_qmm))
            count += 1
    if fuse_siblings:
        _group_siblings(model)
    return count


__all__ = [
    "QuantizedLinear",
    "SiblingGroup",
    "VerifyQuantizedLinear",
    "install_verify_linears",
    "is_verify_eligible",
    "prewarm_verify_kernels",
    "_lib",
]
