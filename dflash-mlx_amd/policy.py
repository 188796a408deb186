"""When the verify path is switched on for a target model.

Restates the reference's load-time gate:

* ``supports_verify_linear`` -- the target-family capability
  (dflash_mlx/engine/target_qwen_gdn.py:811-828): a dense model qualifies
  from 40 layers up; a MoE model qualifies unless it is the one
  40-layer / hidden 2048 / 16 heads / 2 KV heads configuration;
* ``VerifyConfig`` -- mode and qmm switch (dflash_mlx/runtime/__init__.py:30-40);
* ``verify_enabled_for`` / ``verify_qmm_enabled_for`` -- the loader's
  resolution of config vs. DFLASH_VERIFY_LINEAR / DFLASH_VERIFY_QMM
  (dflash_mlx/runtime/loading.py:194-206, 215-230);
* ``install_for_target`` -- the loader's install step: swap the eligible
  linears when both the capability and the mode allow it, and report the
  count the reference stores as ``meta["verify_linear_swapped"]``.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

from . import internal_debug

_MODES = ("dflash", "adaptive", "ddtree", "off")


@dataclass(frozen=True)
class VerifyConfig:
    mode: str = "dflash"
    enable_qmm: bool = True

    @classmethod
    def from_mode(cls, mode: Optional[str]) -> "VerifyConfig":
        resolved = (mode or "dflash").strip().lower()
        if resolved not in _MODES:
            raise ValueError("verify mode must be dflash, adaptive, ddtree, or off")
        return cls(mode=resolved)


def supports_verify_linear(*, num_layers: int, num_experts: int = 0, hidden_size: int = 0,
                           num_heads: int = 0, num_kv_heads: int = 0) -> bool:
    """Target capability: MoE models except (40, 2048, 16, 2); dense from 40 layers."""
    if num_experts > 0:
        for name, v in (("hidden_size", hidden_size), ("num_attention_heads", num_heads),
                        ("num_key_value_heads", num_kv_heads)):
            if int(v) <= 0:
                raise ValueError(f"{name} must be a positive integer for a MoE target")
        return not (num_layers == 40 and hidden_size == 2048 and num_heads == 16
                    and num_kv_heads == 2)
    return num_layers >= 40


def verify_enabled_for(verify_config: Optional[VerifyConfig] = None) -> bool:
    """Config mode wins; without a config DFLASH_VERIFY_LINEAR=0/1 overrides; default on."""
    if verify_config is not None:
        return verify_config.mode != "off"
    override = internal_debug.verify_linear_override()
    return True if override is None else override


def verify_qmm_enabled_for(verify_config: Optional[VerifyConfig] = None) -> bool:
    """Config's enable_qmm; without a config DFLASH_VERIFY_QMM == "1"."""
    if verify_config is not None:
        return bool(verify_config.enable_qmm)
    return internal_debug.verify_qmm_enabled()


def install_for_target(model, *, supports_verify_linear_: bool,
                       verify_config: Optional[VerifyConfig] = None) -> int:
    """Swap the model's eligible linears when the target supports the verify
    path and the mode enables it; returns the number swapped (0 otherwise)."""
    if not (supports_verify_linear_ and verify_enabled_for(verify_config)):
        return 0
    from .verify_linear import install_verify_linears

    return install_verify_linears(model, enable_qmm=verify_qmm_enabled_for(verify_config))
