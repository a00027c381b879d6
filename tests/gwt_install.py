"""Writes synthetic .gwt installations for the loader tests: manifest.json as the
reference's Installer writes it (GodwitManifest, JSONEncoder with sorted keys,
Install/Installer.swift:166-186) and experts/layer_NN.bin files of expertCount
strides each.  The spec object follows the reference's own fixture
(Tests/GodwitTests/TensorNamingTests.swift:90-95)."""
import json
import os

import numpy as np

SECTIONS = ("gate_up_blocks", "gate_up_scales", "down_blocks", "down_scales", "gate_up_bias",
            "down_bias")


def spec_json(hidden, inter, experts, top_k, layers, activation="gptOssClampedGLU",
              eps=1e-5, extra=None):
    spec = {"name": "gpt-oss-test", "hiddenSize": hidden, "intermediateSize": inter,
            "attentionHeads": 64, "keyValueHeads": 8, "headDimension": 64,
            "vocabularySize": 201088, "ropeTheta": 150000, "rmsNormEpsilon": eps,
            "activation": activation, "tiedEmbedding": False, "attentionSinks": True,
            "attentionBias": True, "expertBias": True, "routerBias": True,
            "layers": [{"attention": "full", "window": 0, "routedExpertCount": experts,
                        "expertsPerToken": top_k, "hasSharedExpert": False}
                       for _ in range(layers)]}
    spec.update(extra or {})
    return spec


def write_install(root, layout, layer_blobs, top_k=4, format_version=2, spec=None,
                  drop_section=None):
    """layer_blobs: one uint8 array of layout.stride * expert_count bytes per layer."""
    os.makedirs(os.path.join(root, "experts"), exist_ok=True)
    for l, blob in enumerate(layer_blobs):
        np.asarray(blob, np.uint8).tofile(os.path.join(root, "experts", f"layer_{l:02d}.bin"))
    open(os.path.join(root, "trunk.bin"), "wb").close()
    sections = {n: {"offset": layout.offsets[n], "length": layout.sizes[n]} for n in SECTIONS
                if n != drop_section}
    manifest = {"formatVersion": format_version, "model": "openai/gpt-oss-test",
                "revision": "main",
                "spec": spec or spec_json(layout.hidden_size, layout.intermediate_size,
                                          layout.expert_count, top_k, len(layer_blobs)),
                "layerCount": len(layer_blobs), "expertCount": layout.expert_count,
                "expertStride": layout.stride, "expertSections": sections, "trunkSections": [],
                "bytesWritten": sum(b.size for b in layer_blobs)}
    with open(os.path.join(root, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=2, sort_keys=True)
    return manifest
