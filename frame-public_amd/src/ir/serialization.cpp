// Text form of the IR (format owned by include/frame/ir/serialization.h; it is the reference's format,
// include/frame/ir/serialization.h:1-60, so golden texts and cache keys agree between implementations).
// dump_text walks the topological order; parse_text is a small cursor-based parser that rebuilds the graph
// through the public construction API only.
#include <charconv>
#include <map>
#include <string>
#include <string_view>
#include <system_error>
#include <unordered_map>
#include <utility>
#include <vector>

#include <frame/ir/serialization.h>

namespace frame::ir {

namespace {

std::string dims_text(const Shape& s) {
  std::string out;
  for (size_t i = 0; i < s.dims().size(); ++i) {
    if (i) out += ',';
    out += std::to_string(s.dims()[i]);
  }
  return out;
}

bool reads_as_double(std::string_view t) {
  return t.find_first_of(".eE") != std::string_view::npos || t.find("inf") != std::string_view::npos ||
         t.find("nan") != std::string_view::npos;
}

std::string double_text(double v) {
  char buf[64];
  auto r = std::to_chars(buf, buf + sizeof buf, v);  // shortest round-trip, locale independent
  FRAME_CHECK(r.ec == std::errc());
  std::string t(buf, r.ptr);
  if (!reads_as_double(t)) t += ".0";
  return t;
}

std::string quoted(std::string_view s) {
  std::string out = "\"";
  for (char c : s) {
    if (c == '\\') out += "\\\\";
    else if (c == '"') out += "\\\"";
    else if (c == '\n') out += "\\n";
    else out += c;
  }
  return out + "\"";
}

std::string type_text(const TensorType& t) {
  std::string out = std::string(t.dtype.name()) + "[" + dims_text(t.shape) + "]@" + std::string(t.device.backend) +
                    ":" + std::to_string(t.device.index);
  if (t.layout == Layout::kRowMajor) out += ":row_major";
  return out;
}

template <typename T, typename F>
std::string list_text(const std::vector<T>& v, F&& f) {
  std::string out = "[";
  for (size_t i = 0; i < v.size(); ++i) {
    if (i) out += ", ";
    out += f(v[i]);
  }
  return out + "]";
}

}  // namespace

std::string format_attr_value(const AttrValue& value) {
  return std::visit(
      [](const auto& v) -> std::string {
        using V = std::decay_t<decltype(v)>;
        if constexpr (std::is_same_v<V, int64_t>) return std::to_string(v);
        else if constexpr (std::is_same_v<V, double>) return double_text(v);
        else if constexpr (std::is_same_v<V, std::string>) return quoted(v);
        else if constexpr (std::is_same_v<V, bool>) return v ? "true" : "false";
        else if constexpr (std::is_same_v<V, std::vector<int64_t>>)
          return list_text(v, [](int64_t x) { return std::to_string(x); });
        else if constexpr (std::is_same_v<V, std::vector<double>>) return list_text(v, double_text);
        else if constexpr (std::is_same_v<V, DType>) return "dtype(" + std::string(v.name()) + ")";
        else return "shape[" + dims_text(v) + "]";
      },
      value);
}

std::string dump_text(const Graph& graph) {
  std::unordered_map<const Value*, int64_t> id;
  int64_t next = 0;
  std::string out;
  for (const Node* n : graph.topological_order()) {
    std::string line;
    if (!n->outputs().empty()) {
      for (size_t i = 0; i < n->outputs().size(); ++i) {
        id[&n->outputs()[i]] = next;
        if (i) line += ", ";
        line += "%" + std::to_string(next++);
      }
      line += " = ";
    }
    line += std::string(n->op()) + "(";
    for (size_t i = 0; i < n->inputs().size(); ++i) {
      auto it = id.find(n->inputs()[i]);
      FRAME_CHECK(it != id.end());
      if (i) line += ", ";
      line += "%" + std::to_string(it->second);
    }
    line += ")";
    if (!n->attrs().empty()) {
      std::map<std::string, const AttrValue*> sorted;
      for (const auto& [k, v] : n->attrs()) sorted.emplace(k, &v);
      line += " {";
      bool first = true;
      for (const auto& [k, v] : sorted) {
        if (!first) line += ", ";
        first = false;
        line += k + "=" + format_attr_value(*v);
      }
      line += "}";
    }
    if (!n->outputs().empty()) {
      line += " : ";
      for (size_t i = 0; i < n->outputs().size(); ++i) {
        if (i) line += ", ";
        line += type_text(n->outputs()[i].type());
      }
    }
    out += line + "\n";
  }
  for (const Value* v : graph.outputs()) {
    auto it = id.find(v);
    FRAME_CHECK(it != id.end());
    out += std::string(kGraphOutputMarker) + "(%" + std::to_string(it->second) + ")\n";
  }
  return out;
}

// ---- parser -----------------------------------------------------------------------------------------------

namespace {

class LineParser {
 public:
  LineParser(std::string_view line, int64_t lineno) : s_(line), line_(lineno) {}

  Status error(const std::string& msg) const {
    return Status::make(ErrorCode::kInvalidArgument, "parse_text: line " + std::to_string(line_) + ": " + msg);
  }
  bool eat(std::string_view tok) {
    if (s_.substr(pos_, tok.size()) != tok) return false;
    pos_ += tok.size();
    return true;
  }
  bool at_end() const { return pos_ >= s_.size(); }
  char peek() const { return at_end() ? '\0' : s_[pos_]; }

  // Characters up to (not including) the first top-level occurrence of one of `stops`; brackets, parentheses
  // and quoted strings are skipped as units.
  std::string_view until(std::string_view stops) {
    const size_t start = pos_;
    int depth = 0;
    bool quoted = false;
    while (pos_ < s_.size()) {
      const char c = s_[pos_];
      if (quoted) {
        if (c == '\\' && pos_ + 1 < s_.size()) ++pos_;
        else if (c == '"') quoted = false;
      } else if (depth == 0 && stops.find(c) != std::string_view::npos) {
        break;
      } else if (c == '"') {
        quoted = true;
      } else if (c == '[' || c == '(') {
        ++depth;
      } else if ((c == ']' || c == ')') && depth > 0) {
        --depth;
      }
      ++pos_;
    }
    return s_.substr(start, pos_ - start);
  }

  Result<int64_t> integer(std::string_view t) const {
    int64_t v = 0;
    auto r = std::from_chars(t.data(), t.data() + t.size(), v);
    if (r.ec != std::errc() || r.ptr != t.data() + t.size())
      return error("invalid int64 literal '" + std::string(t) + "'");
    return v;
  }
  Result<double> real(std::string_view t) const {
    double v = 0;
    auto r = std::from_chars(t.data(), t.data() + t.size(), v);
    if (r.ec != std::errc() || r.ptr != t.data() + t.size())
      return error("invalid double literal '" + std::string(t) + "'");
    return v;
  }
  Result<int64_t> ref(std::string_view t) const {
    if (t.empty() || t[0] != '%') return error("value reference '" + std::string(t) + "' must start with '%'");
    return integer(t.substr(1));
  }

  std::string_view rest() const { return s_.substr(pos_); }
  size_t pos_ = 0;

 private:
  std::string_view s_;
  int64_t line_;
};

// Splits at top-level ", " (commas inside [] / () / quotes and commas without a following space stay).
std::vector<std::string_view> split_items(std::string_view s) {
  std::vector<std::string_view> out;
  if (s.empty()) return out;
  int depth = 0;
  bool quoted = false;
  size_t start = 0;
  for (size_t i = 0; i < s.size(); ++i) {
    const char c = s[i];
    if (quoted) {
      if (c == '\\' && i + 1 < s.size()) ++i;
      else if (c == '"') quoted = false;
      continue;
    }
    if (c == '"') quoted = true;
    else if (c == '[' || c == '(') ++depth;
    else if (c == ']' || c == ')') --depth;
    else if (depth == 0 && c == ',' && i + 1 < s.size() && s[i + 1] == ' ') {
      out.push_back(s.substr(start, i - start));
      start = i + 2;
      ++i;
    }
  }
  out.push_back(s.substr(start));
  return out;
}

Result<std::vector<int64_t>> parse_dims(const LineParser& p, std::string_view inner) {
  std::vector<int64_t> dims;
  if (inner.empty()) return dims;
  size_t start = 0;
  while (true) {
    const size_t comma = inner.find(',', start);
    Result<int64_t> d = p.integer(inner.substr(start, comma == std::string_view::npos ? inner.npos : comma - start));
    if (!d.is_ok()) return d.status();
    dims.push_back(d.value());
    if (comma == std::string_view::npos) break;
    start = comma + 1;
  }
  return dims;
}

Result<DType> parse_dtype_name(const LineParser& p, std::string_view name) {
  for (uint8_t c = 0; c < static_cast<uint8_t>(DTypeCode::kCount); ++c)
    if (DType(static_cast<DTypeCode>(c)).name() == name) return DType(static_cast<DTypeCode>(c));
  return p.error("unknown dtype name '" + std::string(name) + "'");
}

Result<std::string_view> known_backend(const LineParser& p, std::string_view name) {
  for (std::string_view b : {kCpuBackendName, kCudaBackendName, kIntelGpuBackendName, kIntelNpuBackendName,
                             kAscendBackendName, kHipBackendName})
    if (name == b) return b;  // static storage: the Device view must not point into the parsed text
  return p.error("unknown backend name '" + std::string(name) + "'");
}

Result<AttrValue> parse_attr(const LineParser& p, std::string_view v) {
  if (!v.empty() && v.front() == '"') {
    if (v.size() < 2 || v.back() != '"') return p.error("malformed string attribute value '" + std::string(v) + "'");
    std::string out;
    for (size_t i = 1; i + 1 < v.size(); ++i) {
      char c = v[i];
      if (c == '\\' && i + 2 < v.size()) {
        const char e = v[++i];
        if (e == 'n') c = '\n';
        else if (e == '\\' || e == '"') c = e;
        else return p.error("unknown escape sequence in string attribute value");
      }
      out += c;
    }
    return AttrValue{std::move(out)};
  }
  if (v.substr(0, 6) == "dtype(") {
    if (v.size() < 7 || v.back() != ')') return p.error("malformed dtype attribute value '" + std::string(v) + "'");
    Result<DType> d = parse_dtype_name(p, v.substr(6, v.size() - 7));
    if (!d.is_ok()) return d.status();
    return AttrValue{d.value()};
  }
  if (v.substr(0, 6) == "shape[") {
    if (v.size() < 7 || v.back() != ']') return p.error("malformed shape attribute value '" + std::string(v) + "'");
    Result<std::vector<int64_t>> d = parse_dims(p, v.substr(6, v.size() - 7));
    if (!d.is_ok()) return d.status();
    return AttrValue{Shape(d.value())};
  }
  if (v == "true") return AttrValue{true};
  if (v == "false") return AttrValue{false};
  if (!v.empty() && v.front() == '[') {
    if (v.size() < 2 || v.back() != ']') return p.error("malformed array attribute value '" + std::string(v) + "'");
    std::vector<std::string_view> items = split_items(v.substr(1, v.size() - 2));
    bool any_double = false;
    for (auto t : items) any_double = any_double || reads_as_double(t);
    if (any_double) {
      std::vector<double> out;
      for (auto t : items) {
        Result<double> d = p.real(t);
        if (!d.is_ok()) return d.status();
        out.push_back(d.value());
      }
      return AttrValue{std::move(out)};
    }
    std::vector<int64_t> out;  // an empty array reads as int64 array
    for (auto t : items) {
      Result<int64_t> d = p.integer(t);
      if (!d.is_ok()) return d.status();
      out.push_back(d.value());
    }
    return AttrValue{std::move(out)};
  }
  if (reads_as_double(v)) {
    Result<double> d = p.real(v);
    if (!d.is_ok()) return d.status();
    return AttrValue{d.value()};
  }
  Result<int64_t> i = p.integer(v);
  if (!i.is_ok()) return i.status();
  return AttrValue{i.value()};
}

Result<TensorType> parse_type(const LineParser& p, std::string_view t) {
  TensorType type;
  constexpr std::string_view kRowMajor = ":row_major";
  if (t.size() > kRowMajor.size() && t.substr(t.size() - kRowMajor.size()) == kRowMajor) {
    type.layout = Layout::kRowMajor;
    t.remove_suffix(kRowMajor.size());
  }
  const size_t lb = t.find('['), rb = t.find(']'), at = t.find('@'), colon = t.rfind(':');
  if (lb == t.npos || rb == t.npos || at == t.npos || colon == t.npos || !(lb < rb && rb < at && at < colon))
    return p.error("malformed tensor type '" + std::string(t) + "'");
  Result<DType> d = parse_dtype_name(p, t.substr(0, lb));
  if (!d.is_ok()) return d.status();
  Result<std::vector<int64_t>> dims = parse_dims(p, t.substr(lb + 1, rb - lb - 1));
  if (!dims.is_ok()) return dims.status();
  Result<std::string_view> b = known_backend(p, t.substr(at + 1, colon - at - 1));
  if (!b.is_ok()) return b.status();
  Result<int64_t> idx = p.integer(t.substr(colon + 1));
  if (!idx.is_ok()) return idx.status();
  type.dtype = d.value();
  type.shape = Shape(dims.value());
  type.device = Device{b.value(), static_cast<int32_t>(idx.value())};
  return type;
}

Status parse_line(std::string_view line, int64_t lineno, std::unordered_map<int64_t, Value*>& ids, Graph& g) {
  LineParser p(line, lineno);
  auto lookup = [&](std::string_view tok) -> Result<Value*> {
    Result<int64_t> r = p.ref(tok);
    if (!r.is_ok()) return r.status();
    auto it = ids.find(r.value());
    if (it == ids.end()) return p.error("reference to undefined value %" + std::to_string(r.value()));
    return it->second;
  };

  const std::string out_prefix = std::string(kGraphOutputMarker) + "(";
  if (line.substr(0, out_prefix.size()) == out_prefix) {
    if (line.back() != ')') return p.error("malformed graph_output line (missing ')')");
    Result<Value*> v = lookup(line.substr(out_prefix.size(), line.size() - out_prefix.size() - 1));
    if (!v.is_ok()) return v.status();
    return g.mark_output(v.value());
  }

  // optional "%a, %b = "
  std::vector<int64_t> lhs;
  const size_t eq = line.find(" = "), paren = line.find('(');
  if (paren == line.npos) return p.error("missing '(' in node definition");
  if (eq != line.npos && eq < paren) {
    for (auto tok : split_items(line.substr(0, eq))) {
      Result<int64_t> r = p.ref(tok);
      if (!r.is_ok()) return r.status();
      lhs.push_back(r.value());
    }
    p.pos_ = eq + 3;
  }
  const std::string_view op = p.until("(");
  if (!p.eat("(")) return p.error("missing '(' after op name");
  const std::string_view args = p.until(")");
  if (!p.eat(")")) return p.error("missing ')' after inputs");
  std::vector<Value*> inputs;
  for (auto tok : split_items(args)) {
    Result<Value*> v = lookup(tok);
    if (!v.is_ok()) return v.status();
    inputs.push_back(v.value());
  }
  std::vector<std::pair<std::string, AttrValue>> attrs;
  if (p.eat(" {")) {
    const std::string_view body = p.until("}");
    if (!p.eat("}")) return p.error("missing '}' after attributes");
    for (auto item : split_items(body)) {
      const size_t e = item.find('=');
      if (e == item.npos) return p.error("malformed attribute (missing '=')");
      Result<AttrValue> v = parse_attr(p, item.substr(e + 1));
      if (!v.is_ok()) return v.status();
      attrs.emplace_back(std::string(item.substr(0, e)), std::move(v.value()));
    }
  }
  std::vector<TensorType> types;
  if (!p.at_end()) {
    if (!p.eat(" : ")) return p.error("malformed trailing output type section");
    for (auto tok : split_items(p.rest())) {
      Result<TensorType> t = parse_type(p, tok);
      if (!t.is_ok()) return t.status();
      types.push_back(t.value());
    }
  }
  if (lhs.size() != types.size()) return p.error("output id count does not match output type count");

  auto bind = [&](int64_t id, Value* v) -> Status {
    if (!ids.emplace(id, v).second) return p.error("duplicate definition of value %" + std::to_string(id));
    return Status::ok();
  };
  if (op == kGraphInputOp) {
    if (types.size() != 1 || !inputs.empty())
      return p.error("graph_input node must have zero inputs and exactly one output");
    Result<Value*> v = g.add_graph_input(types[0]);
    if (!v.is_ok()) return v.status();
    return bind(lhs[0], v.value());
  }
  Result<Node*> n = g.create_node(std::string(op), std::move(inputs), std::move(types));
  if (!n.is_ok()) return n.status();
  for (auto& [k, v] : attrs) n.value()->set_attr(k, std::move(v));
  for (size_t i = 0; i < lhs.size(); ++i) FRAME_RETURN_IF_ERROR(bind(lhs[i], n.value()->output(static_cast<int32_t>(i))));
  return Status::ok();
}

}  // namespace

Result<Graph> parse_text(std::string_view text) {
  Graph g;
  std::unordered_map<int64_t, Value*> ids;
  int64_t lineno = 0;
  size_t start = 0;
  while (start < text.size()) {
    size_t nl = text.find('\n', start);
    if (nl == text.npos) nl = text.size();
    std::string_view line = text.substr(start, nl - start);
    ++lineno;
    start = nl + 1;
    if (line.empty()) continue;
    FRAME_RETURN_IF_ERROR(parse_line(line, lineno, ids, g));
  }
  return g;
}

}  // namespace frame::ir
