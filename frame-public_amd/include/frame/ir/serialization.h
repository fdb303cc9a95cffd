#pragma once
// Deterministic text form of the IR: one line per node
//   %<ids> = <op>(%<in>, ...) {<attr>=<value>, ...} : <dtype>[<d0>,<d1>]@<backend>:<index>[:row_major]
// followed by one `graph_output(%<id>)` line per graph output. Attributes are sorted by name; doubles use the
// shortest round-trip form with ".0" appended when it would read as an integer. The format is the reference's
// (include/frame/ir/serialization.h:1-60): it is the compile-cache key and the golden-test format, and text from
// one implementation parses in the other. parse_text accepts the built-in backend names plus "hip".

#include <string>
#include <string_view>

#include <frame/core/macros.h>
#include <frame/core/status.h>
#include <frame/ir/graph.h>

namespace frame::ir {

FRAME_API std::string format_attr_value(const AttrValue& value);
FRAME_API std::string dump_text(const Graph& graph);
FRAME_API Result<Graph> parse_text(std::string_view text);

}  // namespace frame::ir
