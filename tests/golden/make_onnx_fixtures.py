"""Writes the ONNX importer fixtures under tests/golden/onnx/.

Each fixture is a small seeded PyTorch model exported by torch's TorchScript
ONNX exporter, whose ModelProto bytes come from the ONNX serializer compiled
into libtorch (the onnx Python package is not installed here; the exporter
needs it only to splice custom onnxscript functions into the bytes, and these
models have none, so that step passes the bytes through). Beside each
<name>.onnx, <name>.npz holds the input and the expected output of the same
model evaluated in float64 by torch on the CPU.

    python tests/golden/make_onnx_fixtures.py
"""

from __future__ import annotations

import copy
import io
from pathlib import Path

import numpy as np
import torch
from torch.onnx._internal.torchscript_exporter import onnx_proto_utils

OUT = Path(__file__).resolve().parent / "onnx"


def _passthrough(model_bytes, custom_opsets):
    return model_bytes


class TinyResNet(torch.nn.Module):
    """Stem (7x7/2 conv, BN, ReLU, 3x3/2 max pool), one bottleneck block with
    a projection shortcut, global average pool, flatten, linear."""

    def __init__(self) -> None:
        super().__init__()
        def cbn(cin, cout, k, s=1, p=0):
            return [torch.nn.Conv2d(cin, cout, k, s, p, bias=False), torch.nn.BatchNorm2d(cout)]
        self.stem = torch.nn.Sequential(*cbn(3, 16, 7, 2, 3), torch.nn.ReLU(), torch.nn.MaxPool2d(3, 2, 1))
        self.branch = torch.nn.Sequential(*cbn(16, 8, 1), torch.nn.ReLU(), *cbn(8, 8, 3, 1, 1), torch.nn.ReLU(),
                                          *cbn(8, 32, 1))
        self.shortcut = torch.nn.Sequential(*cbn(16, 32, 1))
        self.fc = torch.nn.Linear(32, 10)
        g = torch.Generator().manual_seed(5)
        for m in self.modules():
            if isinstance(m, torch.nn.BatchNorm2d):  # non-trivial statistics
                m.running_mean.copy_(torch.randn(m.num_features, generator=g) * 0.1)
                m.running_var.copy_(torch.rand(m.num_features, generator=g) + 0.5)
                m.weight.data.copy_(torch.rand(m.num_features, generator=g) + 0.5)
                m.bias.data.copy_(torch.randn(m.num_features, generator=g) * 0.1)

    def forward(self, x):
        x = self.stem(x)
        y = torch.relu(self.branch(x) + self.shortcut(x))
        return self.fc(torch.flatten(torch.nn.functional.adaptive_avg_pool2d(y, 1), 1))


class TinyFfn(torch.nn.Module):
    """Linear -> erf-GELU -> Linear -> residual add -> LayerNorm."""

    def __init__(self, hidden: int = 64, intermediate: int = 256) -> None:
        super().__init__()
        self.fc1 = torch.nn.Linear(hidden, intermediate)
        self.fc2 = torch.nn.Linear(intermediate, hidden)
        self.norm = torch.nn.LayerNorm(hidden)

    def forward(self, x):
        return self.norm(self.fc2(torch.nn.functional.gelu(self.fc1(x))) + x)


def export(model, x, opset, training, dynamic_batch, names):
    f = io.BytesIO()
    torch.onnx.export(model, x, f, dynamo=False, opset_version=opset, training=training,
                      input_names=[names[0]], output_names=[names[1]],
                      dynamic_axes={names[0]: {0: "batch"}, names[1]: {0: "batch"}} if dynamic_batch else None)
    return f.getvalue()


def main() -> None:
    onnx_proto_utils._add_onnxscript_fn = _passthrough
    OUT.mkdir(parents=True, exist_ok=True)
    torch.manual_seed(3)
    cnn = TinyResNet().eval()
    x = torch.randn(2, 3, 32, 32)
    want = copy.deepcopy(cnn).double()(x.double()).detach().numpy()
    for name, mode in (("tiny_resnet_folded", torch.onnx.TrainingMode.EVAL),
                       ("tiny_resnet_batchnorm", torch.onnx.TrainingMode.PRESERVE)):
        (OUT / f"{name}.onnx").write_bytes(export(cnn, x, 17, mode, True, ("input", "output")))
        np.savez(OUT / f"{name}.npz", input=x.numpy(), output=want)
    torch.manual_seed(4)
    ffn = TinyFfn().eval().half()  # the file and the float64 reference share the FP16 weights
    xh = torch.randn(24, 64).half()
    want = copy.deepcopy(ffn).double()(xh.double()).detach().numpy()
    (OUT / "tiny_ffn_fp16.onnx").write_bytes(export(ffn, xh, 20, torch.onnx.TrainingMode.EVAL, False, ("x", "y")))
    np.savez(OUT / "tiny_ffn_fp16.npz", input=xh.numpy(), output=want)
    for p in sorted(OUT.iterdir()):
        print(p.name, p.stat().st_size)


if __name__ == "__main__":
    main()
