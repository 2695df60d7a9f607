"""ONNX files for the importer tests, written by google.protobuf.

The messages are declared here with the field numbers, types and packing of
the public ONNX schema (onnx/onnx.proto, IR version 3 and later; the onnx
package itself is not installed), so the files come from an encoder that
shares no code with the engine's reader. ``to_onnx`` turns a
workloads.GraphSpec into a serialized ModelProto.
"""

from __future__ import annotations

from typing import Any

import numpy as np
from google.protobuf import descriptor_pb2, descriptor_pool, message_factory

F = descriptor_pb2.FieldDescriptorProto
OPT, REP = F.LABEL_OPTIONAL, F.LABEL_REPEATED

# TensorProto.DataType and AttributeProto.AttributeType values.
ONNX_DTYPES = {"float32": 1, "int32": 6, "int64": 7, "float16": 10, "float64": 11}
ATTR_FLOAT, ATTR_INT, ATTR_STRING, ATTR_TENSOR, ATTR_GRAPH, ATTR_FLOATS, ATTR_INTS = 1, 2, 3, 4, 5, 6, 7

# message -> [(field, number, type, label, message type or None, packed)]
SCHEMA: dict[str, list[tuple[str, int, int, int, str | None, bool]]] = {
    "Dimension": [("dim_value", 1, F.TYPE_INT64, OPT, None, False),
                  ("dim_param", 2, F.TYPE_STRING, OPT, None, False)],
    "TensorShapeProto": [("dim", 1, F.TYPE_MESSAGE, REP, "Dimension", False)],
    "TensorType": [("elem_type", 1, F.TYPE_INT32, OPT, None, False),
                   ("shape", 2, F.TYPE_MESSAGE, OPT, "TensorShapeProto", False)],
    "TypeProto": [("tensor_type", 1, F.TYPE_MESSAGE, OPT, "TensorType", False)],
    "ValueInfoProto": [("name", 1, F.TYPE_STRING, OPT, None, False),
                       ("type", 2, F.TYPE_MESSAGE, OPT, "TypeProto", False)],
    "TensorProto": [("dims", 1, F.TYPE_INT64, REP, None, False),
                    ("data_type", 2, F.TYPE_INT32, OPT, None, False),
                    ("float_data", 4, F.TYPE_FLOAT, REP, None, True),
                    ("int32_data", 5, F.TYPE_INT32, REP, None, True),
                    ("int64_data", 7, F.TYPE_INT64, REP, None, True),
                    ("name", 8, F.TYPE_STRING, OPT, None, False),
                    ("raw_data", 9, F.TYPE_BYTES, OPT, None, False),
                    ("double_data", 10, F.TYPE_DOUBLE, REP, None, True),
                    ("data_location", 14, F.TYPE_INT32, OPT, None, False)],
    "AttributeProto": [("name", 1, F.TYPE_STRING, OPT, None, False),
                       ("f", 2, F.TYPE_FLOAT, OPT, None, False),
                       ("i", 3, F.TYPE_INT64, OPT, None, False),
                       ("s", 4, F.TYPE_BYTES, OPT, None, False),
                       ("t", 5, F.TYPE_MESSAGE, OPT, "TensorProto", False),
                       ("g", 6, F.TYPE_MESSAGE, OPT, "GraphProto", False),
                       ("floats", 7, F.TYPE_FLOAT, REP, None, False),
                       ("ints", 8, F.TYPE_INT64, REP, None, False),
                       ("type", 20, F.TYPE_INT32, OPT, None, False)],
    "NodeProto": [("input", 1, F.TYPE_STRING, REP, None, False),
                  ("output", 2, F.TYPE_STRING, REP, None, False),
                  ("name", 3, F.TYPE_STRING, OPT, None, False),
                  ("op_type", 4, F.TYPE_STRING, OPT, None, False),
                  ("attribute", 5, F.TYPE_MESSAGE, REP, "AttributeProto", False),
                  ("domain", 7, F.TYPE_STRING, OPT, None, False)],
    "GraphProto": [("node", 1, F.TYPE_MESSAGE, REP, "NodeProto", False),
                   ("name", 2, F.TYPE_STRING, OPT, None, False),
                   ("initializer", 5, F.TYPE_MESSAGE, REP, "TensorProto", False),
                   ("input", 11, F.TYPE_MESSAGE, REP, "ValueInfoProto", False),
                   ("output", 12, F.TYPE_MESSAGE, REP, "ValueInfoProto", False),
                   ("sparse_initializer", 15, F.TYPE_MESSAGE, REP, "TensorProto", False)],
    "OperatorSetIdProto": [("domain", 1, F.TYPE_STRING, OPT, None, False),
                           ("version", 2, F.TYPE_INT64, OPT, None, False)],
    "ModelProto": [("ir_version", 1, F.TYPE_INT64, OPT, None, False),
                   ("producer_name", 2, F.TYPE_STRING, OPT, None, False),
                   ("graph", 7, F.TYPE_MESSAGE, OPT, "GraphProto", False),
                   ("opset_import", 8, F.TYPE_MESSAGE, REP, "OperatorSetIdProto", False)],
}


def _classes(pack_all: bool) -> dict[str, Any]:
    """Message classes; pack_all packs every repeated scalar (proto3 style)."""
    package = "onnx_test_packed" if pack_all else "onnx_test"
    fdp = descriptor_pb2.FileDescriptorProto(name=package + ".proto", package=package, syntax="proto2")
    for message, fields in SCHEMA.items():
        m = fdp.message_type.add(name=message)
        for name, number, ftype, label, type_name, packed in fields:
            f = m.field.add(name=name, number=number, type=ftype, label=label)
            if type_name:
                f.type_name = f".{package}.{type_name}"
            if label == REP and ftype != F.TYPE_MESSAGE and ftype not in (F.TYPE_STRING, F.TYPE_BYTES):
                f.options.packed = packed or pack_all
    pool = descriptor_pool.DescriptorPool()
    pool.Add(fdp)
    return {name: message_factory.GetMessageClass(pool.FindMessageTypeByName(f"{package}.{name}"))
            for name in SCHEMA}


ONNX = _classes(False)
ONNX_PACKED = _classes(True)


def tensor(cls: dict[str, Any], name: str, array: np.ndarray, raw: bool = True) -> Any:
    """A TensorProto of `array`: raw_data, or the typed field ONNX assigns
    (float_data for FLOAT, int32_data for FLOAT16 bit patterns and INT32,
    int64_data for INT64)."""
    array = np.ascontiguousarray(array)
    t = cls["TensorProto"](name=name, dims=list(array.shape), data_type=ONNX_DTYPES[str(array.dtype)])
    if raw:
        t.raw_data = array.tobytes()
    elif array.dtype == np.float32:
        t.float_data.extend(array.ravel().tolist())
    elif array.dtype == np.float16:
        t.int32_data.extend(array.ravel().view(np.uint16).astype(np.int64).tolist())
    elif array.dtype == np.int32:
        t.int32_data.extend(array.ravel().tolist())
    else:
        t.int64_data.extend(array.ravel().tolist())
    return t


def attribute(cls: dict[str, Any], name: str, value: Any) -> Any:
    a = cls["AttributeProto"](name=name)
    if isinstance(value, bool) or isinstance(value, (int, np.integer)):
        a.type, a.i = ATTR_INT, int(value)
    elif isinstance(value, float):
        a.type, a.f = ATTR_FLOAT, value
    elif isinstance(value, str):
        a.type, a.s = ATTR_STRING, value.encode()
    elif isinstance(value, (list, tuple)) and all(isinstance(v, (int, np.integer)) for v in value):
        a.type = ATTR_INTS
        a.ints.extend(int(v) for v in value)
    elif isinstance(value, (list, tuple)):
        a.type = ATTR_FLOATS
        a.floats.extend(float(v) for v in value)
    else:
        raise TypeError(f"attribute {name}: {value!r}")
    return a


def value_info(cls: dict[str, Any], name: str, shape=None, dtype: str | None = None, symbolic: dict | None = None):
    """ValueInfoProto; `symbolic` maps an axis to a dim_param name."""
    v = cls["ValueInfoProto"](name=name)
    if shape is not None:
        v.type.tensor_type.elem_type = ONNX_DTYPES[dtype]
        for axis, d in enumerate(shape):
            dim = v.type.tensor_type.shape.dim.add()
            if symbolic and axis in symbolic:
                dim.dim_param = symbolic[axis]
            else:
                dim.dim_value = int(d)
    return v


def to_onnx(spec, opset: int = 17, raw: bool = True, packed: bool = False, symbolic: dict | None = None,
            ir_version: int = 8) -> bytes:
    """Serializes `spec` (workloads.GraphSpec) as an ONNX ModelProto.
    `symbolic` maps input name -> {axis: dim_param}."""
    cls = ONNX_PACKED if packed else ONNX
    model = cls["ModelProto"](ir_version=ir_version, producer_name="cutriton_amd tests")
    model.opset_import.add(domain="", version=opset)
    g = model.graph
    g.name = "graph"
    for name, (shape, dtype, _) in spec.inputs.items():
        g.input.append(value_info(cls, name, shape, dtype, (symbolic or {}).get(name)))
    for name, (array, _) in spec.constants.items():
        g.initializer.append(tensor(cls, name, array, raw))
    for node in spec.nodes:
        n = g.node.add(name=node.name, op_type=node.op_type)
        n.input.extend(node.inputs)
        n.output.extend(node.outputs)
        for key, value in node.attributes.items():
            n.attribute.append(attribute(cls, key, value))
    for name in spec.outputs:
        g.output.append(value_info(cls, name))
    return model.SerializeToString()
