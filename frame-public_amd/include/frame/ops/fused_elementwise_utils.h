#pragma once
// Encoding of fused_elementwise_internal nodes (reference: include/frame/ops/fused_elementwise_utils.h:28-73):
// attr "ops" = sub-op names joined by ';' in execution order, attr "arities" = their input counts. Segment 0
// takes the first arities[0] external inputs; segment i > 0 takes the previous segment's result as input 0 and
// the next arities[i]-1 external inputs.

#include <cstdint>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

#include <frame/core/macros.h>
#include <frame/core/status.h>
#include <frame/ir/attribute.h>
#include <frame/ops/kernel_registry.h>

namespace frame::hal {
class Allocator;
}

namespace frame::ops {

inline constexpr std::string_view kFusedElementwiseOpName = "fused_elementwise_internal";

struct FusedElementwiseChain {
  std::vector<std::string> sub_ops;
  std::vector<int64_t> arities;
};

FRAME_API void encode_fused_chain(const std::vector<std::string>& ops, const std::vector<int64_t>& arities,
                                  std::unordered_map<std::string, ir::AttrValue>& attrs);

// Decodes and checks: both attrs present with the right types, equal counts, sum(arities) - (segments - 1) ==
// expected_input_count, every sub-op registered with kElementwise and kFusable.
FRAME_API Status decode_and_validate_fused_chain(const std::unordered_map<std::string, ir::AttrValue>& attrs,
                                                 int64_t expected_input_count, FusedElementwiseChain& out);

// Backend-generic composition: runs each segment through KernelRegistry::find(sub_op, ctx.device.backend) with
// temporaries from `allocator`. Backends with a single-pass kernel (the hip backend) do not use it.
FRAME_API Status execute_fused_chain(const KernelContext& ctx, hal::Allocator& allocator);

}  // namespace frame::ops
