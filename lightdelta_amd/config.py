"""Process-level backend configuration; fails closed on unknown sections, keys and values.

Same fields, defaults, TOML layout and validation rules as the reference's BackendConfig
(python/lightdelta/config.py:8-60), so its configs/*.toml files load unchanged:
  [gdn]         compute = "torch_reference" | "cuda_fused"
                state_io = "packed" | "indexed"
                prefill_io = "reference" | "fused_copy"
  [runtime]     torch_compile (must be false), cuda_graph
  [speculation] method = "none" | "mtp", num_speculative_tokens
On ROCm, "cuda_fused" selects the gfx950 HIP kernels (the name is kept for drop-in configs).
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

try:  # Python >= 3.11
    import tomllib as _toml
except ModuleNotFoundError:  # Python 3.10: the API-identical tomli package
    import tomli as _toml

_SECTIONS = {
    "gdn": {"compute", "state_io", "prefill_io"},
    "runtime": {"torch_compile", "cuda_graph"},
    "speculation": {"method", "num_speculative_tokens"},
}


@dataclass(frozen=True)
class BackendConfig:
    compute: str = "torch_reference"
    state_io: str = "packed"
    prefill_io: str = "reference"
    torch_compile: bool = False
    cuda_graph: bool = False
    speculation_method: str = "none"
    num_speculative_tokens: int = 0

    @classmethod
    def from_file(cls, path: str | Path) -> "BackendConfig":
        return cls.from_toml(Path(path).read_text())

    @classmethod
    def from_toml(cls, text: str) -> "BackendConfig":
        data = _toml.loads(text)
        unknown = data.keys() - _SECTIONS.keys()
        if unknown:
            raise ValueError(f"Unknown config sections: {unknown}")
        for section, values in data.items():
            if not isinstance(values, dict) or values.keys() - _SECTIONS[section]:
                raise ValueError(f"Unknown keys or invalid table in [{section}]")
        speculation = data.get("speculation", {})
        config = cls(
            **data.get("gdn", {}),
            **data.get("runtime", {}),
            speculation_method=speculation.get("method", "none"),
            num_speculative_tokens=speculation.get("num_speculative_tokens", 0),
        )
        config.validate()
        return config

    def validate(self) -> None:
        defaults = BackendConfig()
        for name in self.__dataclass_fields__:
            if type(getattr(self, name)) is not type(getattr(defaults, name)):
                raise ValueError(f"Invalid type for {name}")
        if self.compute not in ("torch_reference", "cuda_fused"):
            raise ValueError("compute must be torch_reference or cuda_fused")
        if self.state_io not in ("packed", "indexed"):
            raise ValueError("state_io must be packed or indexed")
        if self.prefill_io not in ("reference", "fused_copy"):
            raise ValueError("prefill_io must be reference or fused_copy")
        if self.torch_compile:
            raise ValueError("torch.compile is disabled for controlled ablations")
        if self.compute == "torch_reference" and (self.state_io != "packed" or self.cuda_graph):
            raise ValueError("Torch reference requires packed state and eager execution")
        if self.speculation_method == "none":
            if self.num_speculative_tokens != 0:
                raise ValueError("none speculation requires zero draft tokens")
        elif self.speculation_method != "mtp" or self.num_speculative_tokens not in (1, 2, 3):
            raise ValueError("MTP requires 1, 2 or 3 draft tokens")
