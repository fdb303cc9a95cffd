// ONNX initializer codec: a protobuf wire-format writer and a forward-only reader for the few ModelProto fields the
// weight exchange uses (behaviour of the reference's src/interop/onnx_weights.cpp, written for this repository).
//
// Wire format (protobuf): every field is a varint key (field_number << 3 | wire_type) followed by a varint
// (wire 0), 8 bytes (wire 1), a varint length and that many bytes (wire 2), or 4 bytes (wire 5). Fields used:
//   ModelProto   1 ir_version (varint) = 8, 8 opset_import (message), 7 graph (message)
//   OperatorSetIdProto   1 domain (string) = "", 2 version (varint) = 13
//   GraphProto   2 name (string) = "frame_weights", 5 initializer (repeated TensorProto)
//   TensorProto  1 dims (repeated varint, unpacked), 2 data_type (1 FLOAT, 10 FLOAT16, 16 BFLOAT16),
//                8 name (string), 9 raw_data (bytes, little-endian element bytes)
// The writer emits the fields in that order, so a file written here is byte-identical to the reference's.
#include <frame/interop/onnx_weights.h>

#include <bit>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <iterator>
#include <optional>
#include <string_view>

#include <frame/core/device.h>
#include <frame/core/dtype.h>
#include <frame/core/shape.h>

namespace frame::interop {
namespace {

static_assert(std::endian::native == std::endian::little, "raw_data is little-endian element bytes");

enum Wire : uint32_t { kVarint = 0, kFixed64 = 1, kBytes = 2, kGroupStart = 3, kGroupEnd = 4, kFixed32 = 5 };

// ---- writer ----
struct Writer {
  std::string buf;
  void varint(uint64_t v) {
    for (; v >= 0x80; v >>= 7) buf.push_back(static_cast<char>(0x80 | (v & 0x7f)));
    buf.push_back(static_cast<char>(v));
  }
  void key(uint32_t field, Wire w) { varint((static_cast<uint64_t>(field) << 3) | w); }
  void field_varint(uint32_t field, uint64_t v) {
    key(field, kVarint);
    varint(v);
  }
  void field_bytes(uint32_t field, const void* p, size_t n) {
    key(field, kBytes);
    varint(n);
    buf.append(static_cast<const char*>(p), n);
  }
  void field_bytes(uint32_t field, std::string_view s) { field_bytes(field, s.data(), s.size()); }
};

std::optional<uint32_t> onnx_type_of(DType d) {
  switch (d.code()) {
    case DTypeCode::kFloat32: return 1;
    case DTypeCode::kFloat16: return 10;
    case DTypeCode::kBFloat16: return 16;
    default: return std::nullopt;
  }
}

// ---- reader ----
struct Reader {
  std::string_view data;
  size_t pos = 0;
  bool done() const { return pos >= data.size(); }
  Result<uint64_t> varint() {
    uint64_t v = 0;
    for (int shift = 0; shift < 64; shift += 7) {
      if (pos >= data.size())
        return Status::make(ErrorCode::kInvalidArgument, "load_onnx_weights: truncated varint at offset " + std::to_string(pos));
      const uint8_t b = static_cast<uint8_t>(data[pos++]);
      v |= static_cast<uint64_t>(b & 0x7f) << shift;
      if ((b & 0x80) == 0) return v;
    }
    return Status::make(ErrorCode::kInvalidArgument, "load_onnx_weights: varint longer than 64 bits at offset " + std::to_string(pos));
  }
  Result<std::string_view> take(uint64_t n) {
    if (n > data.size() - pos)
      return Status::make(ErrorCode::kInvalidArgument,
                          "load_onnx_weights: field runs past the end of the buffer at offset " + std::to_string(pos));
    std::string_view s = data.substr(pos, static_cast<size_t>(n));
    pos += static_cast<size_t>(n);
    return s;
  }
  Result<std::string_view> bytes() {
    Result<uint64_t> n = varint();
    if (!n.is_ok()) return n.status();
    return take(n.value());
  }
  Status skip(uint32_t wire) {
    switch (wire) {
      case kVarint: return varint().status();
      case kFixed64: return take(8).status();
      case kFixed32: return take(4).status();
      case kBytes: return bytes().status();
      case kGroupStart:
      case kGroupEnd:
        return Status::make(ErrorCode::kUnimplemented, "load_onnx_weights: deprecated group wire type " +
                                                           std::to_string(wire) + " at offset " + std::to_string(pos));
      default:
        return Status::make(ErrorCode::kInvalidArgument,
                            "load_onnx_weights: unknown wire type " + std::to_string(wire) + " at offset " + std::to_string(pos));
    }
  }
};

// Calls on_field(field, wire, reader) for every field of `msg`; on_field returns true when it consumed the value,
// false to have it skipped.
template <typename F>
Status for_each_field(std::string_view msg, F&& on_field) {
  Reader r{msg};
  while (!r.done()) {
    Result<uint64_t> k = r.varint();
    if (!k.is_ok()) return k.status();
    const uint32_t field = static_cast<uint32_t>(k.value() >> 3), wire = static_cast<uint32_t>(k.value() & 7);
    Result<bool> used = on_field(field, wire, r);
    if (!used.is_ok()) return used.status();
    if (!used.value()) FRAME_RETURN_IF_ERROR(r.skip(wire));
  }
  return Status::ok();
}

Result<NamedTensor> read_tensor(std::string_view msg, hal::Allocator& allocator) {
  std::vector<int64_t> dims;
  std::optional<DType> dtype;
  std::string name;
  std::optional<std::string_view> raw;
  Status st = for_each_field(msg, [&](uint32_t field, uint32_t wire, Reader& r) -> Result<bool> {
    if (field == 1 && wire == kVarint) {
      Result<uint64_t> v = r.varint();
      if (!v.is_ok()) return v.status();
      dims.push_back(static_cast<int64_t>(v.value()));
      return true;
    }
    if (field == 2 && wire == kVarint) {
      Result<uint64_t> v = r.varint();
      if (!v.is_ok()) return v.status();
      const int64_t t = static_cast<int64_t>(v.value());
      if (t == 1) dtype = DType(DTypeCode::kFloat32);
      else if (t == 10) dtype = DType(DTypeCode::kFloat16);
      else if (t == 16) dtype = DType(DTypeCode::kBFloat16);
      else
        return Status::make(ErrorCode::kInvalidArgument, "load_onnx_weights: TensorProto.data_type " + std::to_string(t) +
                                                             " is not one of FLOAT=1, FLOAT16=10, BFLOAT16=16");
      return true;
    }
    if (field == 8 && wire == kBytes) {
      Result<std::string_view> v = r.bytes();
      if (!v.is_ok()) return v.status();
      name = std::string(v.value());
      return true;
    }
    if (field == 9 && wire == kBytes) {
      Result<std::string_view> v = r.bytes();
      if (!v.is_ok()) return v.status();
      raw = v.value();
      return true;
    }
    return false;
  });
  if (!st.is_ok()) return st;
  if (!dtype) return Status::make(ErrorCode::kInvalidArgument, "load_onnx_weights: TensorProto '" + name + "' has no data_type");
  Result<Tensor> t = Tensor::empty(Shape(dims), *dtype, cpu_device(), allocator);
  if (!t.is_ok()) return t.status();
  const size_t nbytes = static_cast<size_t>(t.value().numel()) * dtype->itemsize();
  if (!raw) {
    if (nbytes != 0) return Status::make(ErrorCode::kInvalidArgument, "load_onnx_weights: TensorProto '" + name + "' has no raw_data");
  } else if (raw->size() != nbytes) {
    return Status::make(ErrorCode::kInvalidArgument, "load_onnx_weights: TensorProto '" + name + "' raw_data holds " +
                                                         std::to_string(raw->size()) + " bytes, its shape and dtype need " +
                                                         std::to_string(nbytes));
  }
  if (nbytes != 0) std::memcpy(t.value().raw_data(), raw->data(), nbytes);
  return NamedTensor{std::move(name), std::move(t.value())};
}

}  // namespace

Status save_onnx_weights(const std::string& path, std::span<const NamedTensor> weights) {
  Writer graph;
  graph.field_bytes(2, std::string_view("frame_weights"));
  for (const NamedTensor& w : weights) {
    if (w.tensor.device().backend != kCpuBackendName)
      return Status::make(ErrorCode::kInvalidArgument, "save_onnx_weights: tensor '" + w.name + "' is on backend '" +
                                                           std::string(w.tensor.device().backend) + "', not cpu");
    const std::optional<uint32_t> type = onnx_type_of(w.tensor.dtype());
    if (!type)
      return Status::make(ErrorCode::kInvalidArgument, "save_onnx_weights: tensor '" + w.name + "' has dtype '" +
                                                           std::string(w.tensor.dtype().name()) +
                                                           "', not float32, float16 or bfloat16");
    Writer t;
    for (int64_t d : w.tensor.shape().dims()) t.field_varint(1, static_cast<uint64_t>(d));
    t.field_varint(2, *type);
    t.field_bytes(8, std::string_view(w.name));
    t.field_bytes(9, w.tensor.raw_data(), static_cast<size_t>(w.tensor.numel()) * w.tensor.dtype().itemsize());
    graph.field_bytes(5, t.buf);
  }
  Writer opset;
  opset.field_bytes(1, std::string_view(""));
  opset.field_varint(2, 13);
  Writer model;
  model.field_varint(1, 8);
  model.field_bytes(8, opset.buf);
  model.field_bytes(7, graph.buf);
  std::ofstream out(path, std::ios::binary | std::ios::trunc);
  if (!out) return Status::make(ErrorCode::kInvalidArgument, "save_onnx_weights: cannot open '" + path + "' for writing");
  out.write(model.buf.data(), static_cast<std::streamsize>(model.buf.size()));
  if (!out.good()) return Status::make(ErrorCode::kInternal, "save_onnx_weights: writing '" + path + "' failed");
  return Status::ok();
}

Result<std::vector<NamedTensor>> load_onnx_weights(const std::string& path, hal::Allocator& allocator) {
  std::ifstream in(path, std::ios::binary);
  if (!in) return Status::make(ErrorCode::kNotFound, "load_onnx_weights: cannot open '" + path + "'");
  const std::string file((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
  std::optional<std::vector<NamedTensor>> out;
  Status st = for_each_field(file, [&](uint32_t field, uint32_t wire, Reader& r) -> Result<bool> {
    if (field != 7 || wire != kBytes) return false;
    Result<std::string_view> g = r.bytes();
    if (!g.is_ok()) return g.status();
    std::vector<NamedTensor> tensors;
    Status gs = for_each_field(g.value(), [&](uint32_t f, uint32_t w, Reader& gr) -> Result<bool> {
      if (f != 5 || w != kBytes) return false;
      Result<std::string_view> tm = gr.bytes();
      if (!tm.is_ok()) return tm.status();
      Result<NamedTensor> t = read_tensor(tm.value(), allocator);
      if (!t.is_ok()) return t.status();
      tensors.push_back(std::move(t.value()));
      return true;
    });
    if (!gs.is_ok()) return gs;
    out = std::move(tensors);
    return true;
  });
  if (!st.is_ok()) return st;
  if (!out) return Status::make(ErrorCode::kInvalidArgument, "load_onnx_weights: the ModelProto has no graph field");
  return std::move(*out);
}

}  // namespace frame::interop
