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
import warnings
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
    LaunchRecord,
    _kparts_tuning,
    _m4_ksplit_np_shape,
    _resolve_m16_ktmpl_variant,
    current_stream,
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
        object.__setattr__(obj, "_enable_qmm", enable_qmm)
        object.__setattr__(obj, "_call_fn", _build_dispatch(obj, enable_qmm=enable_qmm))
        obj.requires_grad_(False)
        return obj

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._call_fn(x)

    def _apply(self, fn, recurse=True):
        # .to() / .cuda() / .half() replace the buffers: the launch state
        # (packed tensors, pair table, prepared launches) is rebuilt for the
        # new ones, and the module leaves its sibling group (it then launches
        # alone; install_verify_linears groups it again)
        out = super()._apply(fn, recurse)
        if "_call_fn" in self.__dict__:
            object.__setattr__(self, "_call_fn",
                               _build_dispatch(self, enable_qmm=self.__dict__.get("_enable_qmm")))
        return out


_KERNEL_DTYPES = (torch.bfloat16, torch.float16)

_CAPTURE_WARNED = False


def _warn_capture_without_table() -> None:
    """One RuntimeWarning per process for a verify launch captured into a
    graph before its pair table was built (the graph keeps the slower
    table-free launch; prewarm_verify_kernels before capture avoids it)."""
    global _CAPTURE_WARNED
    if not _CAPTURE_WARNED:
        _CAPTURE_WARNED = True
        warnings.warn("a verify linear was captured into a graph before its pair table was "
                      "built: the captured launch runs without the table (same results, "
                      "slower); call prewarm_verify_kernels(model) before capture",
                      RuntimeWarning, stacklevel=3)


class _VerifyState:
    """Launch state of one verify module, built once by ``_build_dispatch``:
    the packed tensors, the (scale, bias) pair table (the module's own
    ``[K/gs][N]`` table, or its column slice of its sibling group's combined
    table, ``stride`` columns per row), the prepared launches per call shape
    and the sibling group it belongs to."""

    __slots__ = ("w", "s", "b", "N", "K", "gs", "bits", "pairs", "pairs_ok", "stride", "recs",
                 "group", "gidx")

    def __init__(self, w, s, b, N, K, gs, bits):
        self.w, self.s, self.b = w, s, b
        self.N, self.K, self.gs, self.bits = N, K, gs, bits
        self.pairs = None
        self.pairs_ok = (s.dtype in _KERNEL_DTYPES and s.device.type == "cuda" and
                         _runtime.pair_shape(16, K, N, gs, bits))
        self.stride = 0
        self.recs = {}
        self.group = None
        self.gidx = 0

    def pair_table(self):
        """The pair table (built on first use; None while a graph is being
        captured before it exists: the launch then runs without it, with the
        same plan and bit-identical results, and a RuntimeWarning says so
        once per process)."""
        if self.pairs is None and self.pairs_ok:
            if torch.cuda.is_current_stream_capturing():
                _warn_capture_without_table()
                return None
            self.pairs = _runtime.build_sb_pairs(self.s, self.b)
        return self.pairs

    def record(self, m: int, st: int, x: torch.Tensor) -> LaunchRecord:
        """The prepared launch of an [m, K] call on stream st."""
        key = (m, st, x.dtype)
        rec = self.recs.get(key)
        if rec is None:
            t = self.pair_table() if m <= 32 else None
            rec = LaunchRecord(m, self.K, x.dtype, x.device, [(self.w, self.s, self.b, t)],
                               self.gs, self.bits, sb_stride=self.stride if t is not None else 0)
            if t is not None or not self.pairs_ok or m > 32:
                self.recs[key] = rec  # (one made without its table is not kept)
        return rec

    def launch(self, x: torch.Tensor, m: int, st: int) -> torch.Tensor:
        """This module's own launch on x: [m, N]."""
        x2 = x.reshape(m, self.K)
        if not x2.is_contiguous() or x2.data_ptr() & 15:
            x2 = _runtime.aligned_contiguous(x2)
        rec = self.recs.get((m, st, x.dtype)) or self.record(m, st, x)
        y = torch.empty((m, self.N), dtype=x.dtype, device=x.device)
        rec.run(x2, (y,), st)
        return y


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
    # (M = 16 and M = 4 are the verify routes, every other M the stock one;
    # on this GPU both are the same kernels and automatic plan)
    # Reference 176-188 picks mma2big_pipe (K_PARTS 8) or mma2big for shapes
    # the K-templated kernels decline; both run the automatic plan here (the
    # K_PARTS values are Metal launch choices), or DFLASH_VERIFY_QMM_KPARTS
    # splits when the user sets it.
    m16_tuning = _kparts_tuning() if (m16_qmm and ktmpl_variant is None) else None

    def _stock(x):
        return quantized_matmul(x, obj.weight, obj.scales, obj.biases, transpose=True,
                                group_size=gs, bits=bits, mode=mode)

    if m16_qmm or m4_qmm:
        state = _VerifyState(_runtime.weight_words(obj.weight),
                             _runtime.aligned_contiguous(obj.scales),
                             _runtime.aligned_contiguous(obj.biases), N, K, gs, bits)
        # the pair table is built with the route, as the reference evaluates
        # the module's tensors at install (verify_linear.py:148-154), so that a
        # graph captured later finds it
        if state.pairs_ok and not torch.cuda.is_current_stream_capturing():
            state.pair_table()
        object.__setattr__(obj, "_verify_state", state)
        # the verify kernels read scales / biases in the activation dtype:
        # other inputs (fp32, mixed dtypes) go to the stock path
        sdt = state.s.dtype if state.s.dtype in _KERNEL_DTYPES else None

        def call(x: torch.Tensor) -> torch.Tensor:
            shp = x.shape
            kx = shp[-1]
            m = x.numel() // kx if kx else 0
            if x.dtype == sdt and x.is_cuda and 0 < m <= 32 and kx == K:
                if m == 16 and m16_tuning is not None:
                    x2 = _runtime.aligned_contiguous(x.reshape(m, kx))
                    y = qmm_launch(x2, state.w, state.s, state.b, N, gs, bits, m16_tuning)
                else:
                    # M = 16 / M = 4 (the verify routes) and the other small M
                    # (the stock route) run the same automatic plan, through
                    # the module's prepared launch or its sibling group's
                    # shared one; alone, bit-identical to verify_matmul /
                    # quantized_matmul on these tensors
                    st = current_stream(x.get_device())
                    grp = state.group
                    y = grp.product(state.gidx, x, m, st) if grp is not None else None
                    if y is None:
                        y = state.launch(x, m, st)
                y = y.view(*shp[:-1], N)
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
    call per unique (K, N, bits, group_size); also builds every verify
    module's pair table and prepared launches and sizes this stream's
    workspace, so that later calls (and graph captures) neither allocate nor
    plan.  Sibling groups are warmed as groups and then reset (the warm-up
    calls leave no outputs pending)."""
    seen: set[tuple] = set()
    groups = {}
    warmed = 0
    for _, m in _leaf_modules(model):
        if not isinstance(m, VerifyQuantizedLinear):
            continue
        state = m.__dict__.get("_verify_state")
        if state is not None:
            state.pair_table()
            if state.group is not None:
                groups[id(state.group)] = state.group
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
    for grp in groups.values():
        grp.warm(input_dtype)
    return warmed


# Sibling projections that read the same input in the decoder layers the
# reference targets (q/k/v of self_attn, gate/up of mlp).
_SIBLING_SETS = (("q_proj", "k_proj", "v_proj"), ("gate_proj", "up_proj"))


class SiblingGroup:
    """Verify modules of one parent that read the same input (q/k/v, gate/up).

    The first member called with an input of at most 32 rows computes the
    product of every active member in one shared-activation launch
    (``dfmi_qmm_run`` on the group's prepared launch, the members' pair
    tables side by side in one combined table); each other member returns
    its own product when it is called with the same tensor object, unchanged
    (same ``_version``) and on the same stream -- in the model's call order,
    with no change to the model code.  The group holds that input until every
    active member has taken its output, so its storage cannot be reused for
    another tensor meanwhile.  A member called with any other input launches
    the group again.

    A member that leaves its output untaken in two launches running (a layer
    that never calls it, e.g. a shared-KV attention calling q_proj only, or
    ``v_proj`` when k == v) drops out of the shared launch and runs its own
    launch when called; with fewer than two active members left the group
    launches nothing.  Every member's result equals ``quantized_matmul_multi``
    over the active members (plus its bias) bit for bit, and is within fp32
    summation order of the member's own launch."""

    def __init__(self, states, fused: Optional[torch.Tensor], stride: int):
        self.states = list(states)
        self.active = tuple(range(len(self.states)))
        self.fused = fused
        self.stride = stride
        self._miss = [0] * len(self.states)
        self._recs: dict = {}
        self._x = None
        self._ver = -1
        self._st = 0
        self._ys: dict = {}

    def reset(self) -> None:
        """Forget any pending outputs (and the held input) and the miss
        counts, and take every member back into the shared launch."""
        self._x, self._ver, self._st, self._ys = None, -1, 0, {}
        self._miss = [0] * len(self.states)
        self.active = tuple(range(len(self.states)))

    def _record(self, m: int, st: int, x: torch.Tensor) -> LaunchRecord:
        key = (m, st, x.dtype, self.active)
        rec = self._recs.get(key)
        if rec is None:
            sts = [self.states[j] for j in self.active]
            first = sts[0]
            tabs = [st_.pair_table() for st_ in sts]
            # the combined table serves the launch of every member (the
            # fused kernel: two or three matrices of fewer than 2^16 rows);
            # otherwise each matrix reads its column slice of it
            if (self.fused is not None and len(self.active) == len(self.states)
                    and 2 <= len(sts) <= 3 and all(q.N < 65536 for q in sts)):
                rec = LaunchRecord(m, first.K, x.dtype, x.device,
                                   [(q.w, q.s, q.b) for q in sts], first.gs, first.bits,
                                   fused=self.fused)
            elif all(t is not None for t in tabs):
                rec = LaunchRecord(m, first.K, x.dtype, x.device,
                                   [(q.w, q.s, q.b, t) for q, t in zip(sts, tabs)], first.gs,
                                   first.bits, sb_stride=self.stride)
            else:
                rec = LaunchRecord(m, first.K, x.dtype, x.device,
                                   [(q.w, q.s, q.b) for q in sts], first.gs, first.bits)
                if any(q.pairs_ok and t is None for q, t in zip(sts, tabs)):
                    return rec  # made while a table is still missing: not kept
            self._recs[key] = rec
        return rec

    def warm(self, dtype: torch.dtype) -> None:
        """Reset (the members' own warm-up calls leave outputs untaken), then
        prepare and run once the shared launch at M=16 and M=4 on the current
        stream, and reset again."""
        self.reset()
        if len(self.active) >= 2:
            first = self.states[self.active[0]]
            dev = first.w.device
            st = current_stream(dev.index if dev.index is not None else
                                torch.cuda.current_device())
            for m in (16, 4):
                x = torch.zeros((m, first.K), dtype=dtype, device=dev)
                rec = self._record(m, st, x)
                rec.run(x, [torch.empty((m, self.states[j].N), dtype=dtype, device=dev)
                             for j in self.active], st)
        self.reset()

    def product(self, idx: int, x: torch.Tensor, m: int, st: int) -> Optional[torch.Tensor]:
        """Member idx's [m, N] product of x, or None when idx is not in the
        shared launch (the member then launches alone)."""
        ys = self._ys
        if ys and self._x is x and self._ver == x._version and self._st == st:
            y = ys.pop(idx, None)
            if y is not None:
                self._miss[idx] = 0
                if not ys:
                    self._x = None  # every output taken: let the input go
                return y
        if idx not in self.active:
            return None
        if ys:  # members that did not take the previous launch's output
            keep = []
            for j in self.active:
                if j in ys:
                    self._miss[j] += 1
                if self._miss[j] < 2:
                    keep.append(j)
            self.active = tuple(keep) if len(keep) >= 2 else ()
            self._ys = {}
            if idx not in self.active:
                self._x = None
                return None
        x2 = x.reshape(m, int(x.shape[-1]))
        if not x2.is_contiguous() or x2.data_ptr() & 15:
            x2 = _runtime.aligned_contiguous(x2)
        rec = self._recs.get((m, st, x.dtype, self.active)) or self._record(m, st, x)
        outs = [torch.empty((m, self.states[j].N), dtype=x.dtype, device=x.device)
                for j in self.active]
        rec.run(x2, outs, st)
        ys = dict(zip(self.active, outs))
        y = ys.pop(idx)
        self._miss[idx] = 0
        self._ys = ys
        self._x, self._ver, self._st = (x, x._version, st) if ys else (None, -1, 0)
        return y


def _group_siblings(model: nn.Module) -> int:
    """Attach a SiblingGroup to each set of sibling verify modules of one
    parent that share K, bits, group size and scale dtype and take the verify
    kernels; returns the number of groups.  Where the members have pair
    tables, their tables are concatenated into the group's combined table
    and each member keeps only its column slice of it (one copy of the
    scale data per group)."""
    groups = 0
    for _, parent in model.named_modules():
        for names in _SIBLING_SETS:
            mods = [getattr(parent, n, None) for n in names]
            if not all(isinstance(m, VerifyQuantizedLinear) and "_verify_state" in m.__dict__
                       for m in mods):
                continue
            states = [m._verify_state for m in mods]
            sig = {(q.K, q.bits, q.gs, q.s.dtype, q.s.device) for q in states}
            if len(sig) != 1:
                continue
            for q in states:  # a member of an earlier group leaves it
                q.group = None
            fused, stride = None, 0
            tabs = [q.pair_table() for q in states]
            if all(t is not None for t in tabs) and all(q.N % 4 == 0 for q in states):
                # (a member regrouped contributes its column slice of its old
                # group's table)
                fused = torch.cat(tabs, dim=1).contiguous()
                stride = int(fused.shape[1])
                c = 0
                for q in states:  # the members' own tables are released
                    q.pairs = fused[:, c:c + q.N]
                    q.stride = stride
                    q.recs = {}
                    c += q.N
            grp = SiblingGroup(states, fused, stride)
            for i, q in enumerate(states):
                q.group, q.gidx = grp, i
            groups += 1
    return groups


def install_verify_linears(model: nn.Module, *,
                           predicate: Optional[Callable[[str, QuantizedLinear], bool]] = None,
                           enable_qmm: Optional[bool] = None,
                           fuse_siblings: bool = True) -> int:
    """dflash_mlx/verify_linear.py:338-361: swap eligible QuantizedLinear
    leaves for VerifyQuantizedLinear; returns the number swapped.

    ``fuse_siblings`` (no reference counterpart; on by default): group q/k/v
    and gate/up siblings so each set runs as one shared-activation launch
    (:class:`SiblingGroup`); every member's output equals what
    ``quantized_matmul_multi`` returns for it (plus its bias), which is
    within fp32 summation order of the member's own launch.  ``False`` keeps
    one launch per module, each bit-identical to ``verify_matmul``."""
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
