// graph.hpp -- lazy IR graph, compiled plan and executor (graph.cpp).
#pragma once

#include <map>
#include <memory>
#include <string>
#include <vector>

#include "common.hpp"
#include "runtime.hpp"

namespace clove {

// Symbolic dimension: SymInt (backend.rs:30-69) over S0..S3.
struct SymExpr;
using SymPtr = std::shared_ptr<SymExpr>;
struct SymExpr {
    enum { CONST, SYM, ADD, SUB, MUL };
    int kind = CONST;
    int64_t value = 0;  // constant, or symbol index for SYM
    SymPtr a, b;
    int64_t eval(const int64_t *env) const;
    std::string str() const;
    static SymPtr constant(int64_t v);
    static SymPtr binop(int kind, SymPtr a, SymPtr b);
};

std::vector<SymPtr> parse_shape(const std::string &spec);

// IRNode (backend.rs:131-137).
struct Node {
    int id = 0;
    int op = 0;
    std::vector<SymPtr> shape;
    std::vector<int> deps;
    float param = 0.f;
    int64_t pos_offset = 0, head_dim = 0;  // RoPE(pos_offset, head_dim) only
};

// ComputeGraph (backend.rs:149-160), held explicitly instead of in a
// thread-local (lazy.rs:30-33).
struct Graph {
    std::vector<Node> nodes;
    std::vector<int> input_order;
    int add_input(const std::string &spec);
    int add_op(int op, const std::vector<int> &deps, float param);
    int add_rope(int x, int64_t pos_offset, int64_t head_dim);
};

// Step (lazy.rs:1158-1376), hot-path kinds only.
struct Step {
    enum Kind { FUSED, MATMUL, SOFTMAX, LAYER_NORM, PAGED, MATMUL_GROUP, ROPE, ATTENTION };
    Kind kind = FUSED;
    std::vector<int> in;    // node ids read (each once)
    std::vector<int> out;   // node ids written
    std::vector<ChainOp> chain;  // FUSED only
    SymPtr numel;                // FUSED only: index space
    int act = 0;                 // MATMUL only: fused activation (0 none, 1 ReLU, 2 GELU,
                                 // 3 row softmax); a third input, when present, is the
                                 // fused bias
    std::vector<Step> members;   // MATMUL_GROUP only: independent MATMUL steps
    // ROPE: rotation of in[0] at pos_offset q_pos with head_dim.
    // ATTENTION (in = q, k, v): causal attention on row indices with q
    // rotated at q_pos and k at k_pos (head_dim-wide heads), softmax scale
    // `scale` (<= 0: 1/sqrt(head_dim)).
    int64_t q_pos = 0, k_pos = 0, head_dim = 0;
    float scale = 0.f;
};

// CompiledModel (lazy.rs:2545-2555).
struct Model {
    std::vector<Node> nodes;
    std::vector<int> inputs, outputs;
    std::vector<Step> steps;
    std::map<int, int> vbuf;  // node id -> virtual buffer
    int num_vbufs = 0;
    int folded = 0;
    int live_nodes = 0;
    std::vector<TensorNode> buffers;
    std::string description;

    Model(const Graph &g, const std::vector<int> &outs);
    std::string describe() const;
    std::vector<TensorNode> execute(const std::vector<TensorNode> &in, const int64_t *env);
};

}  // namespace clove
