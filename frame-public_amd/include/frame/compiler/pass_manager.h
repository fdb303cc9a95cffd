#pragma once
// PassManager: runs passes in order and verifies the graph after each one
// (reference: include/frame/compiler/pass_manager.h:22-64).

#include <iosfwd>
#include <memory>
#include <string>
#include <string_view>
#include <vector>

#include <frame/compiler/pass.h>
#include <frame/core/macros.h>
#include <frame/core/status.h>

namespace frame::ir {
class Graph;
}

namespace frame::compiler {

class FRAME_API PassManager {
 public:
  PassManager() = default;
  PassManager& add_pass(std::unique_ptr<Pass> pass);
  PassManager& add(std::string_view pass_name);  // a lookup failure is reported by run()
  // Each pass: run, optional IR dump, then graph.verify(make_op_query()); errors are prefixed "pass '<name>': ".
  Status run(ir::Graph& graph) const;
  void set_dump_ir_after(std::string_view pass_name, std::ostream& os);
  std::vector<std::string_view> pass_names() const;

 private:
  std::vector<std::unique_ptr<Pass>> passes_;
  Status pending_error_;
  std::string dump_pass_name_;
  std::ostream* dump_stream_ = nullptr;
};

}  // namespace frame::compiler
