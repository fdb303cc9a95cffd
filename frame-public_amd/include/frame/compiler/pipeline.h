#pragma once
// The fixed standard pipeline (reference: include/frame/compiler/pipeline.h, src/compiler/pipeline.cpp:15-21):
//   canonicalize -> shape_inference -> constant_folding -> common_subexpression_elimination
//   -> dead_node_elimination -> layout_assignment -> operator_fusion -> memory_planning -> backend_lowering

#include <string_view>

#include <frame/compiler/pass_manager.h>
#include <frame/core/macros.h>
#include <frame/core/status.h>

namespace frame::compiler {

FRAME_API Result<PassManager> standard_pipeline(std::string_view backend);

}  // namespace frame::compiler
