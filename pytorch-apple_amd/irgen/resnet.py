"""ResNet-50 (torchvision v1.5 layout) as IR, traced op by op (cfg5).

The reference exports torchvision models through ``torch_ir.extract_ir`` (absent
here); its CUDA path lowers ``aten.conv2d.default``, ``aten.batch_norm.default``,
``aten.relu.default``, ``aten.max_pool2d.default``, ``aten.adaptive_avg_pool2d.default``
and ``aten.linear.default`` (`cuda_compiler/subgraph_analyzer.py:226-369`). This
builder emits the same op sequence an eval-mode export of
``torchvision.models.resnet50`` produces: stem conv 7x7/2 + BN + ReLU + max-pool
3x3/2, four stages of [3, 4, 6, 3] bottlenecks (1x1, 3x3 with the stage stride,
1x1 x4; a 1x1 strided conv + BN on the identity path of each stage's first block),
global average pool, flatten and the 2048 -> 1000 classifier. State-dict keys
follow torchvision (``layer1.0.conv1.weight``, ``bn1.running_mean`` ...).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from irgen.builder import IRBuilder, T


@dataclass(frozen=True)
class ResNetConfig:
    layers: tuple = (3, 4, 6, 3)
    widths: tuple = (64, 128, 256, 512)
    expansion: int = 4
    classes: int = 1000
    eps: float = 1e-5
    dtype: str = "float16"


RESNET50 = ResNetConfig()


def conv(b: IRBuilder, x: T, key: str, cout: int, k: int, stride: int, pad: int, dt: str) -> T:
    w = b.weight(key + ".weight", [cout, x.shape[1], k, k], dt)
    return b.op("aten.conv2d.default", [x, w], {"stride": [stride, stride], "padding": [pad, pad],
                                                "dilation": [1, 1], "groups": 1})


def bn(b: IRBuilder, x: T, key: str, eps: float, dt: str) -> T:
    c = x.shape[1]
    ws = [b.weight(key + ".weight", [c], dt), b.weight(key + ".bias", [c], dt),
          b.weight(key + ".running_mean", [c], dt, buffer=True), b.weight(key + ".running_var", [c], dt, buffer=True)]
    return b.op("aten.batch_norm.default", [x] + ws,
                {"training": False, "momentum": 0.1, "eps": eps, "cudnn_enabled": True})


def relu(b: IRBuilder, x: T) -> T:
    return b.op("aten.relu.default", [x])


def bottleneck(b: IRBuilder, cfg: ResNetConfig, x: T, key: str, width: int, stride: int, down: bool) -> T:
    dt, eps = cfg.dtype, cfg.eps
    out = relu(b, bn(b, conv(b, x, key + ".conv1", width, 1, 1, 0, dt), key + ".bn1", eps, dt))
    out = relu(b, bn(b, conv(b, out, key + ".conv2", width, 3, stride, 1, dt), key + ".bn2", eps, dt))
    out = bn(b, conv(b, out, key + ".conv3", width * cfg.expansion, 1, 1, 0, dt), key + ".bn3", eps, dt)
    idn = x
    if down:
        idn = bn(b, conv(b, x, key + ".downsample.0", width * cfg.expansion, 1, stride, 0, dt),
                 key + ".downsample.1", eps, dt)
    return relu(b, b.op("aten.add.Tensor", [out, idn]))


def build_resnet50_ir(batch: int, image: int = 224, cfg: ResNetConfig = RESNET50) -> dict:
    """cfg5: ``batch`` x 3 x ``image`` x ``image`` -> logits [batch, classes]."""
    b = IRBuilder("ResNet50")
    dt = cfg.dtype
    x = b.input("x", [batch, 3, image, image], dt)
    h = relu(b, bn(b, conv(b, x, "conv1", 64, 7, 2, 3, dt), "bn1", cfg.eps, dt))
    h = b.op("aten.max_pool2d.default", [h], {"kernel_size": [3, 3], "stride": [2, 2], "padding": [1, 1],
                                              "dilation": [1, 1], "ceil_mode": False})
    for si, (n, width) in enumerate(zip(cfg.layers, cfg.widths)):
        for bi in range(n):
            stride = 2 if (bi == 0 and si > 0) else 1
            h = bottleneck(b, cfg, h, f"layer{si + 1}.{bi}", width, stride, down=(bi == 0))
    h = b.op("aten.adaptive_avg_pool2d.default", [h], {"output_size": [1, 1]})
    h = b.op("aten.flatten.using_ints", [h], {"start_dim": 1, "end_dim": -1})
    w = b.weight("fc.weight", [cfg.classes, h.shape[1]], dt)
    bias = b.weight("fc.bias", [cfg.classes], dt)
    b.output(b.op("aten.linear.default", [h, w, bias]))
    return b.to_dict()


_TD = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}


def resnet_weights(ir: dict, seed: int = 0, device: str = "cpu") -> dict[str, torch.Tensor]:
    """He-normal conv weights (std sqrt(2 / fan_in)), BN gamma 1, beta 0, running mean ~N(0, 0.1),
    running var ~U(0.5, 1.5); fc ~N(0, 0.01), bias 0. Drawn in fp32, then cast."""
    g = torch.Generator(device=device).manual_seed(seed)
    out: dict[str, torch.Tensor] = {}
    for w in ir["weights"]:
        key, shape, dt = w["name"], tuple(w["shape"]), _TD[w["dtype"]]
        if key.endswith("running_mean"):
            t = 0.1 * torch.randn(shape, generator=g, device=device)
        elif key.endswith("running_var"):
            t = 0.5 + torch.rand(shape, generator=g, device=device)
        elif len(shape) == 4:
            fan_in = shape[1] * shape[2] * shape[3]
            t = (2.0 / fan_in) ** 0.5 * torch.randn(shape, generator=g, device=device)
        elif key.startswith("fc.") and len(shape) == 2:
            t = 0.01 * torch.randn(shape, generator=g, device=device)
        elif key.endswith(".weight"):
            t = torch.ones(shape, device=device)
        else:
            t = torch.zeros(shape, device=device)
        out[key] = t.to(dt)
    return out


def resnet_inputs(batch: int, image: int = 224, dtype: str = "float16", seed: int = 1,
                  device: str = "cpu") -> dict[str, torch.Tensor]:
    g = torch.Generator(device=device).manual_seed(seed)
    return {"x": torch.randn((batch, 3, image, image), generator=g, device=device).to(_TD[dtype])}
