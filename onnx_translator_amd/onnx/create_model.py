"""ONNX models for the graph path, written with :mod:`onnx_translator_amd.onnx.proto`.

* :func:`comprehensive_model` — the reference's ``create_model.py`` test model,
  ``z = Cos(Relu(x) + Abs(y))`` with x [1,3,32,32] and y [1,1,1,32] (the
  reference exports it with ``torch.onnx.export``, which needs the ``onnx``
  package; here the same graph is written directly, opset 17).
* :func:`woq_gemm_model` — the config-3 weight-only-quantized Gemm:
  ``Gemm(A, DequantizeLinear(Bq, s, zp, axis=0), C, transB=1)`` with A f32
  [256, 4096], Bq int8 [4096, 4096] quantized per output row with scale
  max|B_n| / 127 and zero point 0, and C f32 [4096] (seed 2).
* :func:`resnet_qdq_model` — the QDQ ResNet-style graph: a conv 7x7 / stride 2
  stem with Relu, MaxPool 3x3 / stride 2, four QDQ conv 3x3 blocks (uint8
  per-tensor activations, int8 per-output-channel weights, Relu, residual Add;
  a quantized 1x1 projection where the shape changes), GlobalAveragePool,
  Flatten, Gemm 512 -> 1000 and Softmax over axis 1.  Weights are random
  (He-normal, seeded) and quantized per output channel with scale
  max|w_c| / 127; activations, all non-negative here, use scale 8 / 255 and
  zero point 0.

    python -m onnx_translator_amd.onnx.create_model out.onnx [--batch 64]
"""
from __future__ import annotations

import argparse

import numpy as np

from .proto import (FLOAT, INT8, INT64, UINT8, GraphProto, ModelProto, NodeProto, TensorProto, ValueInfoProto,
                    make_attribute, save)


class _Builder:
    def __init__(self):
        self.nodes, self.inits, self.vinfo = [], [], []

    def init(self, name, arr, dt):
        self.inits.append(TensorProto.from_numpy(arr, name, dt))
        return name

    def node(self, op, ins, outs, **attrs):
        self.nodes.append(NodeProto(op, list(ins), list(outs), name=f"/{op}_{len(self.nodes)}",
                                    attributes=[make_attribute(k, v) for k, v in attrs.items()]))
        return outs[0]

    def typed(self, name, elem, shape=None):
        self.vinfo.append(ValueInfoProto(name, elem, shape))


def comprehensive_model() -> ModelProto:
    b = _Builder()
    b.node("Relu", ["input_x"], ["/relu/Relu_output_0"])
    b.node("Abs", ["input_y"], ["/Abs_output_0"])
    b.node("Add", ["/relu/Relu_output_0", "/Abs_output_0"], ["/Add_output_0"])
    b.node("Cos", ["/Add_output_0"], ["output"])
    g = GraphProto("main_graph", b.nodes, [], [ValueInfoProto("input_x", FLOAT, [1, 3, 32, 32]),
                                               ValueInfoProto("input_y", FLOAT, [1, 1, 1, 32])],
                   [ValueInfoProto("output", FLOAT, [1, 3, 32, 32])])
    return ModelProto(g, producer_name="onnx_translator_amd")


def reshape_model(batch: int = 2) -> ModelProto:
    """``y = Reshape(Relu(x), [batch, -1])`` then ``Cos``: x f32 [batch, 4, 6, 6], the
    target shape an int64 initializer (exercises value-dependent shapes in the graph)."""
    b = _Builder()
    b.init("target", np.array([batch, -1], np.int64), INT64)
    b.node("Relu", ["x"], ["r"])
    b.node("Reshape", ["r", "target"], ["flat"])
    b.node("Cos", ["flat"], ["y"])
    g = GraphProto("reshape_graph", b.nodes, b.inits, [ValueInfoProto("x", FLOAT, [batch, 4, 6, 6])],
                   [ValueInfoProto("y", FLOAT, [batch, 144])])
    return ModelProto(g, producer_name="onnx_translator_amd")


def _quantized_weight(b: _Builder, rng, prefix, shape):
    fan = int(np.prod(shape[1:]))
    w = rng.normal(0, np.sqrt(2.0 / fan), shape)
    s = (np.abs(w).reshape(shape[0], -1).max(axis=1) / 127).astype(np.float32)
    q = np.clip(np.rint(w / s.reshape(-1, *([1] * (len(shape) - 1)))), -127, 127).astype(np.int8)
    b.init(prefix + ".wq", q, INT8)
    b.init(prefix + ".ws", s, FLOAT)
    b.init(prefix + ".wz", np.zeros(shape[0], np.int8), INT8)
    return b.node("DequantizeLinear", [prefix + ".wq", prefix + ".ws", prefix + ".wz"], [prefix + ".w"], axis=0)


def woq_gemm_model(M: int = 256, N: int = 4096, K: int = 4096, seed: int = 2) -> ModelProto:
    rng = np.random.default_rng(seed)
    b = _Builder()
    bw = rng.normal(0, 1 / np.sqrt(K), (N, K))
    s = (np.abs(bw).max(axis=1) / 127).astype(np.float32)
    q = np.clip(np.rint(bw / s[:, None]), -127, 127).astype(np.int8)
    b.init("fc.wq", q, INT8)
    b.init("fc.ws", s, FLOAT)
    b.init("fc.wz", np.zeros(N, np.int8), INT8)
    b.init("fc.b", rng.normal(0, 1 / 64, N).astype(np.float32), FLOAT)
    w = b.node("DequantizeLinear", ["fc.wq", "fc.ws", "fc.wz"], ["fc.w"], axis=0)
    b.node("Gemm", ["input", w, "fc.b"], ["output"], alpha=1.0, beta=1.0, transB=1)
    graph = GraphProto("woq_gemm", b.nodes, b.inits, [ValueInfoProto("input", FLOAT, [M, K])],
                       [ValueInfoProto("output", FLOAT, [M, N])], b.vinfo)
    return ModelProto(graph, producer_name="onnx_translator_amd")


def resnet_qdq_model(batch: int = 64, image: int = 224, seed: int = 4, classes: int = 1000,
                     widths=(64, 128, 256, 512)) -> ModelProto:
    rng = np.random.default_rng(seed)
    b = _Builder()
    b.init("stem.w", rng.normal(0, np.sqrt(2.0 / 147), (widths[0], 3, 7, 7)).astype(np.float32), FLOAT)
    b.init("stem.b", rng.normal(0, 1 / 64, widths[0]).astype(np.float32), FLOAT)
    b.node("Conv", ["input", "stem.w", "stem.b"], ["stem.conv"], dilations=[1, 1], group=1, kernel_shape=[7, 7],
           pads=[3, 3, 3, 3], strides=[2, 2])
    b.node("Relu", ["stem.conv"], ["stem.relu"])
    x = b.node("MaxPool", ["stem.relu"], ["pool"], kernel_shape=[3, 3], pads=[1, 1, 1, 1], strides=[2, 2])
    b.init("act.scale", np.array(8.0 / 255, np.float32), FLOAT)
    b.init("act.zp", np.array(0, np.uint8), UINT8)
    cin = widths[0]
    for i, (cout, stride) in enumerate(zip(widths, (1, 2, 2, 2))):
        p = f"block{i + 1}"
        xq = b.node("QuantizeLinear", [x, "act.scale", "act.zp"], [p + ".xq"])
        b.typed(xq, UINT8)
        xd = b.node("DequantizeLinear", [xq, "act.scale", "act.zp"], [p + ".xd"])
        w = _quantized_weight(b, rng, p, (cout, cin, 3, 3))
        b.init(p + ".b", rng.normal(0, 1 / 64, cout).astype(np.float32), FLOAT)
        conv = b.node("Conv", [xd, w, p + ".b"], [p + ".conv"], dilations=[1, 1], group=1, kernel_shape=[3, 3],
                      pads=[1, 1, 1, 1], strides=[stride, stride])
        h = b.node("Relu", [conv], [p + ".relu"])
        if cin == cout and stride == 1:
            skip = x
        else:
            wp = _quantized_weight(b, rng, p + ".proj", (cout, cin, 1, 1))
            skip = b.node("Conv", [xd, wp], [p + ".proj"], dilations=[1, 1], group=1, kernel_shape=[1, 1],
                          pads=[0, 0, 0, 0], strides=[stride, stride])
        x = b.node("Add", [h, skip], [p + ".out"])
        cin = cout
    g = b.node("GlobalAveragePool", [x], ["gap"])
    f = b.node("Flatten", [g], ["flat"], axis=1)
    b.init("fc.w", rng.normal(0, 1 / np.sqrt(cin), (classes, cin)).astype(np.float32), FLOAT)
    b.init("fc.b", rng.normal(0, 1 / 64, classes).astype(np.float32), FLOAT)
    lg = b.node("Gemm", [f, "fc.w", "fc.b"], ["logits"], alpha=1.0, beta=1.0, transB=1)
    b.node("Softmax", [lg], ["output"], axis=1)
    graph = GraphProto("resnet_qdq", b.nodes, b.inits, [ValueInfoProto("input", FLOAT, [batch, 3, image, image])],
                       [ValueInfoProto("output", FLOAT, [batch, classes])], b.vinfo)
    return ModelProto(graph, producer_name="onnx_translator_amd")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("out")
    ap.add_argument("--model", choices=["resnet_qdq", "woq_gemm", "comprehensive"], default="resnet_qdq")
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--image", type=int, default=224)
    args = ap.parse_args()
    m = {"resnet_qdq": lambda: resnet_qdq_model(args.batch, args.image), "woq_gemm": woq_gemm_model,
         "comprehensive": comprehensive_model}[args.model]()
    save(m, args.out)
    print(f"wrote {args.out}: {len(m.graph.nodes)} nodes, {len(m.graph.initializers)} initializers")


if __name__ == "__main__":
    main()
