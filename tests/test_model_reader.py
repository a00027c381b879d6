"""The .gwt loader's host side (gw_model_open / _info_get / _validate): manifest
parsing and validation as ModelReader.init and GodwitManifest.validate do it
(Runtime/ModelReader.swift:17-37, Install/GodwitManifest.swift:79-104),
including their error messages.  No GPU: these calls only read files."""
import json
import os

import numpy as np
import pytest

import godwit_amd as gw
from gwt_install import spec_json, write_install
from helpers import rng


def _small(tmp_path, layers=2, **kw):
    layout = gw.ExpertLayout(256, 128, 4)
    r = rng(3000)
    blobs = [r.integers(0, 256, layout.stride * 4, dtype=np.uint8) for _ in range(layers)]
    write_install(str(tmp_path), layout, blobs, **kw)
    return layout, blobs


def test_manifest_fields(tmp_path):
    layout, _ = _small(tmp_path, top_k=3)
    m = gw.ModelReader(str(tmp_path))
    assert (m.format_version, m.layer_count, m.expert_count) == (2, 2, 4)
    assert m.expert_stride == layout.stride
    assert m.sections == {n: (layout.offsets[n], layout.sizes[n]) for n in layout.offsets}
    assert (m.hidden_size, m.intermediate_size, m.experts_per_token) == (256, 128, 3)
    assert m.activation == "gptOssClampedGLU" and m.expert_bias and m.router_bias
    assert m.rms_norm_epsilon == pytest.approx(1e-5, rel=1e-6)
    # fields an older install lacks take the decoder's defaults (ArchitectureSpec.swift:176-205)
    assert m.activation_limit == pytest.approx(7.0) and m.activation_alpha == pytest.approx(1.702)
    m.validate()
    m.close()


def test_manifest_spec_overrides_and_qwen3(tmp_path):
    layout = gw.ExpertLayout(256, 128, 4)
    spec = spec_json(256, 128, 4, 8, 1, activation="silu", eps=1e-6,
                     extra={"activationLimit": 5.0, "activationAlpha": 2.0, "expertBias": False,
                            "routerBias": False})
    write_install(str(tmp_path), layout, [np.zeros(layout.stride * 4, np.uint8)], spec=spec)
    m = gw.ModelReader(str(tmp_path))
    assert m.activation == "silu" and m.experts_per_token == 8
    assert (m.activation_limit, m.activation_alpha) == (5.0, 2.0)
    assert not m.expert_bias and not m.router_bias
    m.close()


def test_validate_catches_a_truncated_layer(tmp_path):
    layout, blobs = _small(tmp_path)
    path = os.path.join(str(tmp_path), "experts", "layer_01.bin")
    blobs[1][:-100].tofile(path)
    m = gw.ModelReader(str(tmp_path))
    with pytest.raises(gw.GodwitError, match=r"layer 1 is \d+ bytes, expected \d+"):
        m.validate()
    m.close()


def test_open_errors(tmp_path):
    with pytest.raises(gw.GodwitError, match="no such directory"):
        gw.ModelReader(str(tmp_path / "missing"))
    with pytest.raises(gw.GodwitError, match="has no manifest.json"):
        gw.ModelReader(str(tmp_path))
    _small(tmp_path, format_version=1)
    with pytest.raises(gw.GodwitError, match="format v1, runtime expects v2"):
        gw.ModelReader(str(tmp_path))


def test_missing_section_and_bad_json(tmp_path):
    _small(tmp_path, drop_section="down_bias")
    with pytest.raises(gw.GodwitError, match="manifest has no section 'down_bias'"):
        gw.ModelReader(str(tmp_path))
    with open(os.path.join(str(tmp_path), "manifest.json"), "w") as f:
        f.write('{"formatVersion": 2, "layerCount": ')
    with pytest.raises(gw.GodwitError, match="not valid JSON"):
        gw.ModelReader(str(tmp_path))


def test_parses_the_reference_encoders_layout(tmp_path):
    """Pretty-printed with sorted keys, escapes and nested arrays: the parser reads what
    JSONEncoder writes, and key order does not matter."""
    layout, _ = _small(tmp_path)
    p = os.path.join(str(tmp_path), "manifest.json")
    doc = json.load(open(p))
    doc["model"] = "openai/gpt\\u2011oss \"120b\""
    doc["trunkSections"] = [{"name": "embed", "offset": 0, "length": 16, "dtype": "int8",
                             "shape": [4, 4]}]
    with open(p, "w") as f:
        f.write(json.dumps(doc, indent=4, sort_keys=False, ensure_ascii=True))
    m = gw.ModelReader(str(tmp_path))
    assert m.expert_stride == layout.stride
    m.close()
