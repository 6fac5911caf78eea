// fusion.hpp — FusionAST node types (optimizer/fusion_ast.go:30-65) and the
// HIP codegen target's entry points.
#ifndef MFH_FUSION_HPP
#define MFH_FUSION_HPP

#include <cstdint>

#include "common.hpp"

namespace mfh {

// optimizer.NodeType values, in the Go iota order.
enum NodeType : int32_t {
    kNodeInvalid = 0, kNodeInput, kNodeConstant,
    kNodeAdd, kNodeSub, kNodeMul, kNodeDiv, kNodeMax, kNodeMin,
    kNodeNeg, kNodeAbs, kNodeSqrt, kNodeExp, kNodeLog,
    kNodeReLU, kNodeSigmoid, kNodeTanh, kNodeSilu, kNodeGelu, kNodeLeakyReLU,
};

// NodeType.Arity (optimizer/fusion_ast.go:168-180); -1 for unknown types.
int node_arity(int type);

// EmitHIP and HIPKernel.Run behind mfh_fusion_compile / mfh_fusion_launch.
int emit_hip(const mfh_ast_node* nodes, int n_nodes, const mfh_operand* inputs, int n_inputs,
             uint8_t out_dtype, const char* output_port, uint32_t flags, mfh_kernel** out);
// With may_load false a kernel whose module is not loaded on the current
// device fails instead of being loaded (loading allocates device memory).
int run_hip(const mfh_kernel* kernel, const void* const* inputs, int n_inputs, void* out, int64_t count,
            hipStream_t stream, bool may_load = true);
// Changes whenever a loaded kernel module is unloaded (shutdown, device
// change); function handles taken before a change may be dangling.
uint64_t module_generation();

}  // namespace mfh

#endif  // MFH_FUSION_HPP
