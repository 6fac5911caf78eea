// fusion.hpp — FusionAST node types (optimizer/fusion_ast.go:30-65) and the
// HIP codegen target's entry points.
#ifndef MFH_FUSION_HPP
#define MFH_FUSION_HPP

#include <cstdint>
#include <vector>

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

// The launch run_hip makes: function, grid and argument values.  grid 0 means
// nothing to launch (count 0).
struct HipLaunch {
    hipFunction_t fn = nullptr;
    unsigned grid = 0;
    unsigned block = 0;
    std::vector<const void*> ptrs;  // the inputs
    void* out = nullptr;
    int64_t count = 0;
    int64_t nvec = 0;
    std::vector<void*> args;  // kernel argument addresses, set by bind()
    // Points `args` at the fields above; call it where the object stays
    // until the launch (or node update) has read them.
    void bind();
};
// run_hip's checks and launch shape for these buffers, without the launch.
int prepare_hip(const mfh_kernel* kernel, const void* const* inputs, int n_inputs, void* out, int64_t count,
                bool may_load, HipLaunch* launch);

}  // namespace mfh

#endif  // MFH_FUSION_HPP
