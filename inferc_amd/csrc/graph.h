// The graph IR shared by the ONNX reader, the fusion passes and the
// executor: ir::Graph / ir::Node / ir::Tensor (src/ir/graph.h:40-97) in this
// library's own form. Not part of the C-ABI.
//
//  - Initializers keep their bytes (little-endian, C order).
//  - Node attributes of scalar and list type are kept as text: integers in
//    decimal, floats with 9 significant digits (exact for float32), lists
//    comma-separated, strings as they are. Tensor attributes (Constant's and
//    ConstantOfShape's "value") are kept as initializer records.
//  - Graph inputs carry their declared dtype and shape (-1 = symbolic dim).
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

struct inferc_graph {
  struct Init {
    std::string name;
    int dtype = 0;
    std::vector<int64_t> shape;
    std::vector<uint8_t> data;
  };
  struct Node {
    std::string op, name, domain;
    std::vector<std::string> in, out;
    std::map<std::string, std::string> attrs;
    std::map<std::string, Init> tattrs;
  };
  struct IO {
    std::string name;
    int dtype = 0;
    std::vector<int64_t> shape;
  };
  std::string name;
  std::vector<Init> inits;
  std::vector<Node> nodes;
  std::vector<IO> inputs;
  std::vector<std::string> outputs;
};
