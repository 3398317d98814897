"""BackendConfig: the reference's TOML layout loads unchanged and invalid configs fail closed
(reference python/lightdelta/config.py:8-60)."""

from __future__ import annotations

import pytest

from lightdelta_amd.config import BackendConfig


def toml(compute="cuda_fused", state_io="indexed", prefill_io="reference", graph=True,
         method="mtp", spec=3):
    return f"""
[gdn]
compute = "{compute}"
state_io = "{state_io}"
prefill_io = "{prefill_io}"

[runtime]
torch_compile = false
cuda_graph = {str(graph).lower()}

[speculation]
method = "{method}"
num_speculative_tokens = {spec}
"""


@pytest.mark.parametrize("text,expected", [
    (toml(), BackendConfig("cuda_fused", "indexed", "reference", False, True, "mtp", 3)),
    (toml(state_io="packed", graph=False, method="none", spec=0),
     BackendConfig("cuda_fused", "packed", "reference", False, False, "none", 0)),
    (toml("torch_reference", "packed", graph=False, method="none", spec=0), BackendConfig()),
    (toml(prefill_io="fused_copy"),
     BackendConfig("cuda_fused", "indexed", "fused_copy", False, True, "mtp", 3)),
    ("[gdn]\ncompute = \"cuda_fused\"\n", BackendConfig(compute="cuda_fused")),
])
def test_valid_configs(text, expected):
    assert BackendConfig.from_toml(text) == expected


def test_from_file(tmp_path):
    path = tmp_path / "full.toml"
    path.write_text(toml())
    assert BackendConfig.from_file(path).num_speculative_tokens == 3


@pytest.mark.parametrize("text,message", [
    ("[extra]\nx = 1\n", "Unknown config sections"),
    ("[gdn]\nkernel = \"x\"\n", "Unknown keys"),
    ("gdn = 3\n", "Unknown keys or invalid table"),
    (toml(compute="triton"), "compute must be"),
    (toml(state_io="paged"), "state_io must be"),
    (toml(prefill_io="chunked"), "prefill_io must be"),
    (toml().replace("torch_compile = false", "torch_compile = true"), "torch.compile"),
    (toml("torch_reference", "indexed"), "Torch reference requires packed"),
    (toml("torch_reference", "packed", graph=True), "Torch reference requires packed"),
    (toml(method="none", spec=2), "zero draft tokens"),
    (toml(spec=4), "MTP requires"),
    (toml(method="eagle", spec=1), "MTP requires"),
    (toml().replace("cuda_graph = true", "cuda_graph = 1"), "Invalid type"),
])
def test_invalid_configs_fail_closed(text, message):
    with pytest.raises(ValueError, match=message):
        BackendConfig.from_toml(text)
