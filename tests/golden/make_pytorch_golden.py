"""Writes the fixtures that pin the model-version 12-17 functions of the
oracle and the device path against the reference's own PyTorch model.

Run in a container where /root/reference exists (the tests never read it):
    python tests/golden/make_pytorch_golden.py

What these nets exercise that KataGo's C++ test records (model versions 5 to
11) do not: the two- and four-channel policy outputs mixed by policyOptimism
(eigenbackend.cpp:2539-2549), the version-15 pass MLP (linear_pass, bias,
activation, linear_pass2), fixed 2-D RoPE (model_pytorch.py:1223-1261) and
learnable RoPE (:1263-1290) with grouped-query attention
(TransformerAttentionBlock, :1979-2320), the transformer RMSNorm and the
SwiGLU and plain FFN (TransformerFFNBlock, :2322-2418), transformer blocks
nested in bottleneck blocks (:1853-1977), the per-position and spatial
RMSNorm trunk tips (RMSNormMask, :181-256) and the single batch norm of the
"fson" nets.

For each net the script
  * builds the reference's Model (model_pytorch.py:2808) from a config of
    modelconfigs.py (a named one, or one with fewer blocks or channels, noted
    below), seeds torch, runs Model.initialize(), then moves every parameter
    off the values initialisation leaves trivial (zero-initialised fixup
    convs and biases, unit norm gains; the batch norm's running statistics)
    with a seeded perturbation, so that no layer is an identity;
  * writes the model file with the reference's own exporter
    (python/export_model_pytorch.py, -export-random-initialized-model, run
    through runpy in this process; the Model it builds is captured when its
    initialize() runs, so the forward below uses exactly the weights the
    exporter wrote);
  * runs the reference's forward (trunk in float64, heads in the float32
    its forward casts to) on 16 positions featurized by
    KataGo's own fillRowV7 (from featurize_golden.json.gz, all in 19x19
    tensors: 19x19, 19x11, 17x19, 7x15 and 9x9 boards), and stores the raw
    head outputs in the order the C++ backends read them: the policy channels
    the exporter writes (0 and 5, or 0, 5, 6 and 7), the three value logits,
    the six score channels (misc 0-3 and more-misc 0-1) and the ownership;
    and, from the forward's ExtraOutputs, the trunk after the embedding,
    after each block and after the tip, summarised as KataGo's debug build
    prints it (count, min, max, mean, rms over on-board positions).

Outputs: pytorch_golden_<name>.bin.gz (the exported model) and
pytorch_golden.npz (inputs and outputs, plain arrays, loadable with
allow_pickle=False).
"""
from __future__ import annotations

import copy
import gzip
import json
import math
import os
import runpy
import shutil
import sys
import tempfile

import numpy as np

REF_PY = "/root/reference/python"
HERE = os.path.dirname(os.path.abspath(__file__))

# (fixture name, base config in modelconfigs.py, changes, seed).
NETS = [
    # Version-15 conv net: fixup blocks with gpool, mish, the single batch
    # norm at the trunk tip ("fson"), pass MLP, two policy channels.
    ("b4c32-fson-mish", "b4c32-fson-mish", {}, 11),
    # Version 17: fixed 2-D RoPE with three heads of 16, SwiGLU FFN,
    # per-position RMSNorm tip with SiLU ("rnh"), four policy channels
    # (predict_q_values). b5c48h3tfr with three blocks, and SwiGLU in place
    # of its plain FFN, which KataGo's model format cannot describe (no
    # activation is written for it; eigenbackend.cpp:1621-1622 rejects it).
    ("b3c48h3tfrs-silu-rnh-q", "b5c48h3tfr-silu-rnh",
     {"predict_q_values": True,
      "block_kind": [[f"{k}{i}", kind] for i in (1, 2, 3) for k, kind in (("attn", "attnrope"), ("ffn", "ffnsg"))]}, 12),
    # Version 17: grouped-query attention (6 query heads over 3 KV heads,
    # query dim 32, value dim 16), learnable RoPE, SwiGLU, spatial RMSNorm
    # tip with SiLU ("rsnh"); the reference config's first four of fourteen
    # blocks.
    ("b2c96h6kv3qk32v16tflrs-silu-rsnh", "b7c96h6kv3qk32v16tflrs-silu-rsnh", {"blocks": 4}, 13),
    # Version 17: transformer blocks nested in bottleneck blocks
    # (bottlenest2transformerropesg), fixed RoPE, a gpool conv block, mish,
    # spatial RMSNorm tip; b5c192h3nbttfrs shrunk to 64/32 channels, two
    # heads of 16 and two outer blocks. Its tip activation is mish, where
    # KataGo's backends differ (EIGEN_TIP_IDENTITY below).
    ("b3c64h2nbttfrs-mish-rsnh", "b5c192h3nbttfrs-mish-rsnh",
     {"trunk_num_channels": 64, "mid_num_channels": 32, "gpool_num_channels": 16, "transformer_ffn_channels": 64,
      "transformer_heads": 2, "transformer_kv_heads": 2,
      "block_kind": [["block1", "bottlenest2transformerropesg"], ["rconv2", "regulargpool"],
                     ["block3", "bottlenest2transformerropesg"]]}, 14),
]

# After an RMSNorm trunk tip, KataGo's Eigen backend applies the tip
# activation only if it is SiLU and otherwise none (RMSNormLayer::apply,
# eigenbackend.cpp:982-984,1012-1014), while the CUDA backend applies ReLU,
# Mish or SiLU (cudahelpers.cu:3008-3010), the OpenCL backend rejects any
# other than SiLU (openclbackend.cpp:2117-2119) and the PyTorch model applies
# the configured one (model_pytorch.py:3664-3665). For these nets the
# fixture's outputs follow the Eigen backend (the forward runs with
# act_trunkfinal replaced by identity); the outputs of the unmodified
# forward are stored beside them under "<name>/model_act/...".
EIGEN_TIP_IDENTITY = {"b3c64h2nbttfrs-mish-rsnh"}

# Positions of the featurizer fixture, all in 19x19 tensors: eight 19x19
# boards and two each of 19x11, 17x19, 7x15 and 9x9.
BOARDS = [((19, 19), 8), ((19, 11), 2), ((17, 19), 2), ((7, 15), 2), ((9, 9), 2)]
OPTIMISM = [0.0, 0.5, 1.0]


def positions():
    with gzip.open(os.path.join(HERE, "featurize_golden.json.gz"), "rt") as f:
        fx = json.load(f)["positions"]
    chosen = []
    for (x, y), count in BOARDS:
        rows = [p for p in fx if p["nnx"] == 19 and p["nny"] == 19 and p["x_size"] == x and p["y_size"] == y]
        # Spread over the games: later positions carry more history planes.
        step = max(1, len(rows) // count)
        chosen += rows[::step][:count]
    assert len(chosen) == 16
    spatial = np.zeros((16, 19 * 19 * 22), np.uint8)
    glob = np.zeros((16, 19), np.float32)
    for i, p in enumerate(chosen):
        bits = bin(int(p["spatial_nhwc_bits"], 16))[2:].zfill(len(p["spatial_nhwc_bits"]) * 4)
        spatial[i] = np.frombuffer(bits[:19 * 19 * 22].encode(), np.uint8) - ord("0")
        glob[i] = p["global"]
    return spatial, glob


def perturb(model, seed):
    """Moves parameters off the trivial values initialisation leaves."""
    import torch
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if bool(torch.all(p == 0)):
                if name.endswith("weight") and p.dim() >= 2:
                    fan_in = p[0].numel()
                    p.copy_(torch.randn(p.shape, generator=g, dtype=p.dtype) * (0.5 / math.sqrt(fan_in)))
                else:
                    p.copy_(torch.randn(p.shape, generator=g, dtype=p.dtype) * 0.1)
            elif bool(torch.all(p == 1)):
                p.mul_(0.75 + 0.5 * torch.rand(p.shape, generator=g, dtype=p.dtype))
        for m in model.modules():
            if getattr(m, "is_using_batchnorm", False):
                m.running_mean.copy_(torch.randn(m.running_mean.shape, generator=g) * 0.1)
                m.running_std.copy_(0.8 + 0.4 * torch.rand(m.running_std.shape, generator=g))


def export_and_forward(name, base, changes, seed, spatial_nhwc, glob, tmp):
    import torch
    from katago.train import modelconfigs
    import katago.train.model_pytorch as mp

    cfg = copy.deepcopy(modelconfigs.config_of_name[base])
    if "blocks" in changes:
        cfg["block_kind"] = cfg["block_kind"][:changes["blocks"]]
    cfg.update({k: v for k, v in changes.items() if k != "blocks"})
    modelconfigs.config_of_name[name] = cfg

    captured = []
    orig_init = mp.Model.initialize

    def initialize_and_perturb(self):
        orig_init(self)
        perturb(self, seed + 1000)
        captured.append(self)

    mp.Model.initialize = initialize_and_perturb
    argv = sys.argv
    try:
        torch.manual_seed(seed)
        sys.argv = ["export_model_pytorch.py", "-export-random-initialized-model", name, "-export-dir", tmp,
                    "-model-name", name, "-filename-prefix", name]
        runpy.run_path(os.path.join(REF_PY, "export_model_pytorch.py"), run_name="__main__")
    finally:
        sys.argv = argv
        mp.Model.initialize = orig_init
    assert len(captured) == 1
    model = captured[0]
    with open(os.path.join(tmp, name + ".bin"), "rb") as f, gzip.GzipFile(
            os.path.join(HERE, f"pytorch_golden_{name}.bin.gz"), "wb", compresslevel=9, mtime=0) as g:
        shutil.copyfileobj(f, g)

    model.eval()
    # The trunk in float64; the heads stay float32, since the reference's
    # forward casts the trunk output to float32 for them (model_pytorch.py:3671-3676).
    model.double()
    model.policy_head.float()
    model.value_head.float()
    n = spatial_nhwc.shape[0]
    x = torch.tensor(spatial_nhwc.reshape(n, 19, 19, 22).transpose(0, 3, 1, 2).astype(np.float64))
    gl = torch.tensor(glob.astype(np.float64))

    nblocks = len(model.blocks)
    names = ["trunk_after_embedding"] + [f"trunk_after_block{i}" for i in range(nblocks)] + ["trunkfinal"]
    on = x[:, 0:1, :, :].numpy() > 0

    def heads():
        eo = mp.ExtraOutputs(names)
        with torch.no_grad():
            out = model(x, gl, extra_outputs=eo)[0]
        policy, value, misc, moremisc, ownership = (t.numpy() for t in out[:5])
        # The trunk before each block, after the last and after the tip, as
        # KataGo's debug build summarises them: element count, min, max, mean
        # and root mean square over on-board positions, all channels.
        stats = []
        for nm in names:
            t = eo.returned[nm].numpy()
            v = t[np.broadcast_to(on, t.shape)]
            stats.append([v.size, v.min(), v.max(), v.mean(), np.sqrt((v * v).mean())])
        chans = [0, 5] if policy.shape[1] == 6 else [0, 5, 6, 7]
        return {
            "policy": policy[:, chans, :],  # [n][channels][361 + pass]
            "value": value,  # [n][3]
            "score": np.concatenate([misc[:, 0:4], moremisc[:, 0:2]], axis=1),
            "ownership": ownership.reshape(n, 361),
            "trunkstats": np.array(stats, np.float64),
        }

    result = heads()
    if name in EIGEN_TIP_IDENTITY:
        result["model_act"] = result
        model.act_trunkfinal = torch.nn.Identity()
        result = dict(heads(), model_act=result["model_act"])
    return result


def main():
    sys.path.insert(0, REF_PY)
    spatial, glob = positions()
    arrays = {"spatial_nhwc": spatial, "global": glob, "optimism": np.array(OPTIMISM, np.float32)}
    names = []
    with tempfile.TemporaryDirectory() as tmp:
        for name, base, changes, seed in NETS:
            r = export_and_forward(name, base, changes, seed, spatial, glob, tmp)
            for k in ("policy", "value", "score", "ownership", "trunkstats"):
                arrays[f"{name}/{k}"] = r[k]
                if "model_act" in r:
                    arrays[f"{name}/model_act/{k}"] = r["model_act"][k]
            names.append(name)
            print(name, "policy channels", r["policy"].shape[1], "value[0]", r["value"][0])
    arrays["names"] = np.array(names)
    np.savez_compressed(os.path.join(HERE, "pytorch_golden.npz"), **arrays)


if __name__ == "__main__":
    main()
