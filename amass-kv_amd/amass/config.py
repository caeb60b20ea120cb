"""AmassConfig -- the single source of truth for AMASS behaviour (drop-in surface).

Same field set, defaults, validation and ``AMASS_CONFIG`` loading rules as the
reference's ``src/amass/config.py:26-165``: a frozen dataclass built once (from an
optional ``AMASS_CONFIG`` that is a JSON/YAML file path or an inline JSON string, plus
explicit overrides); unknown keys raise.  Kernels never read the environment.

Variants: ``fast`` (K+V resident), ``mem-v`` (V in a pinned host tier), ``mem-kv``.
On this MI355X build, ``coverage`` drives a per-(request, kv-head) nucleus on the
score-derived page masses whenever ``budget`` is None (the reference's graph-safe path
falls back to a fixed 10% budget there, ``backend/builder.py:192-194``).
"""
from __future__ import annotations

import dataclasses
import json
import os
from typing import Literal, Optional

Variant = Literal["fast", "mem-v", "mem-kv"]
Table = Literal["kv-union", "q-head", "kv-shared"]


@dataclasses.dataclass(frozen=True)
class AmassConfig:
    # ---- variant -------------------------------------------------------------- #
    variant: Variant = "mem-v"
    # ---- Stage A: decode-time page selection ---------------------------------- #
    coverage: float = 0.95          # per-head nucleus coverage (used when budget is None)
    budget: Optional[float] = None  # fixed selected fraction; overrides coverage
    table: Table = "kv-union"
    sink_pages: int = 1
    window_pages: int = 1
    r8_screen: bool = False
    r8_rank: int = 8
    score: Literal["r8", "quad", "clse"] = "clse"
    quad_rank: int = 2
    quad_v_bits: int = 4
    quad_combine: Literal["max", "nrm"] = "nrm"
    quad_c_bits: int = 4
    quad_c_grain: Literal["token", "page"] = "token"
    # ---- Stage B / tier -------------------------------------------------------- #
    hot_slots: int = 2048
    v_blocks: Optional[int] = None
    max_pool_gb: float = 256.0
    # ---- engine / kernels ------------------------------------------------------ #
    use_cuda: bool = True           # kept for config compatibility: the HIP kernels
    force_eager: bool = False       # are the only implementation on this build

    @property
    def is_mem(self) -> bool:
        return self.variant in ("mem-v", "mem-kv")

    @property
    def offload_k(self) -> bool:
        return self.variant == "mem-kv"

    def __post_init__(self) -> None:
        if self.variant not in ("fast", "mem-v", "mem-kv"):
            raise ValueError(f"unknown variant {self.variant!r}")
        if self.offload_k and not self.r8_screen:
            object.__setattr__(self, "r8_screen", True)
        if not (0.0 < self.coverage <= 1.0):
            raise ValueError(f"coverage must be in (0,1], got {self.coverage}")
        if self.budget is not None and not (0.0 < self.budget <= 1.0):
            raise ValueError(f"budget must be in (0,1], got {self.budget}")
        if self.score not in ("r8", "quad", "clse"):
            raise ValueError(f"score must be 'r8', 'quad' or 'clse', got {self.score!r}")
        if self.quad_rank < 1:
            raise ValueError(f"quad_rank must be >= 1, got {self.quad_rank}")
        if self.quad_v_bits not in (4, 8):
            raise ValueError(f"quad_v_bits must be 4 or 8, got {self.quad_v_bits}")
        if self.quad_combine not in ("max", "nrm"):
            raise ValueError(
                f"quad_combine must be 'max' or 'nrm', got {self.quad_combine!r}")
        if self.quad_c_bits not in (4, 8):
            raise ValueError(f"quad_c_bits must be 4 or 8, got {self.quad_c_bits}")
        if self.quad_c_grain not in ("token", "page"):
            raise ValueError(
                f"quad_c_grain must be 'token' or 'page', got {self.quad_c_grain!r}")

    @classmethod
    def load(cls, overrides: Optional[dict] = None) -> "AmassConfig":
        """Build from the optional ``AMASS_CONFIG`` (file path or inline JSON) plus
        explicit ``overrides``; the only place configuration is read from the env."""
        data: dict = {}
        spec = os.environ.get("AMASS_CONFIG")
        if spec:
            if os.path.isfile(spec):
                with open(spec) as fh:
                    text = fh.read()
                if spec.endswith((".yaml", ".yml")):
                    import yaml
                    data = yaml.safe_load(text) or {}
                else:
                    data = json.loads(text)
            else:
                data = json.loads(spec)
        if overrides:
            data.update({k: v for k, v in overrides.items() if v is not None})
        fields = {f.name for f in dataclasses.fields(cls)}
        unknown = set(data) - fields
        if unknown:
            raise ValueError(f"unknown AmassConfig keys: {sorted(unknown)}")
        return cls(**data)
