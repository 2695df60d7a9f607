// ONNX model import: a native reader of the ONNX protobuf format into a
// Model. The reference has no importer (its Python facade only lists the
// structure of a model through the onnx package, python/cutriton/api.py:77-99,
// and README.md:338 lists the importer as missing); this one needs no
// protobuf or onnx library.
//
// What is read:
//   * graph inputs that are not initializers become model inputs (layout
//     "NCHW" at rank 4, "" otherwise);
//   * initializers and Constant nodes become host constants (FLOAT, FLOAT16,
//     INT32, INT64; raw_data or the typed fields);
//   * nodes of the default domain keep their op_type, inputs, outputs and
//     INT, INTS, FLOAT, FLOATS and STRING attributes (a node without a name
//     is named "<op_type>_<index>");
//   * graph outputs become model outputs.
// Refused (InvalidArgument for malformed data, Unsupported otherwise):
// external or sparse tensor data, graph-valued attributes, nodes of other
// domains, and attribute values whose meaning the engine's ops would drop
// silently: Conv group != 1 or auto_pad other than NOTSET, MaxPool
// ceil_mode = 1, Gemm alpha or beta != 1, Gelu approximate = "tanh".
// Softmax without an axis below opset 13 gets axis 1, that opset's default.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>

#include "cutriton/core/status.h"
#include "cutriton/ir/graph.h"

namespace cutriton {

// Sizes for symbolic input dimensions (dim_param name -> size). An input
// dimension that is symbolic and not named here is an error.
using OnnxDimValues = std::unordered_map<std::string, int64_t>;

// Reads a serialized ONNX ModelProto from memory into `model` (which must be
// empty).
Status ImportOnnxModel(const void* data, std::size_t size, const OnnxDimValues& dim_values, Model* model);

// Reads the ONNX file at `path` into `model`.
Status ImportOnnxFile(const std::string& path, const OnnxDimValues& dim_values, Model* model);

}  // namespace cutriton
