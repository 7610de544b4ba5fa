// Safetensors reader for the weight loader (src/gpu/weights.rs:28-319):
// 8-byte little-endian header length, JSON header of
// {name: {dtype, shape, data_offsets}}, then the raw tensor bytes.
#include <cctype>
#include <cstring>
#include <fstream>

#include "runtime.h"

namespace ppocr {
namespace {

class Json {
 public:
  explicit Json(const std::string& s) : s_(s) {}
  void ws() {
    while (i_ < s_.size() && isspace((unsigned char)s_[i_])) ++i_;
  }
  char peek() {
    ws();
    if (i_ >= s_.size()) raise(PPOCR_ERR_SAFETENSORS, "decode safetensors: truncated header");
    return s_[i_];
  }
  bool eat(char c) {
    if (peek() == c) {
      ++i_;
      return true;
    }
    return false;
  }
  void expect(char c) {
    if (!eat(c)) raise(PPOCR_ERR_SAFETENSORS, std::string("decode safetensors: expected '") + c + "'");
  }
  std::string str() {
    expect('"');
    std::string out;
    while (i_ < s_.size() && s_[i_] != '"') {
      if (s_[i_] == '\\' && i_ + 1 < s_.size()) ++i_;
      out.push_back(s_[i_++]);
    }
    if (i_ >= s_.size()) raise(PPOCR_ERR_SAFETENSORS, "decode safetensors: unterminated string");
    ++i_;
    return out;
  }
  uint64_t uint() {
    ws();
    if (i_ >= s_.size() || !isdigit((unsigned char)s_[i_]))
      raise(PPOCR_ERR_SAFETENSORS, "decode safetensors: expected an unsigned integer");
    uint64_t v = 0;
    while (i_ < s_.size() && isdigit((unsigned char)s_[i_])) {
      uint64_t d = (uint64_t)(s_[i_++] - '0');
      if (v > (UINT64_MAX - d) / 10) raise(PPOCR_ERR_SAFETENSORS, "decode safetensors: integer overflow");
      v = v * 10 + d;
    }
    return v;
  }
  void skip() {
    char c = peek();
    if (c == '"') {
      str();
    } else if (c == '{') {
      ++i_;
      if (eat('}')) return;
      do {
        str();
        expect(':');
        skip();
      } while (eat(','));
      expect('}');
    } else if (c == '[') {
      ++i_;
      if (eat(']')) return;
      do skip();
      while (eat(','));
      expect(']');
    } else {
      while (i_ < s_.size() && !strchr(",}] \n\r\t", s_[i_])) ++i_;
    }
  }

 private:
  const std::string& s_;
  size_t i_ = 0;
};

}  // namespace

SafeTensors SafeTensors::load(const std::string& path) {
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  if (!f) raise(PPOCR_ERR_READ_FILE, "read weights " + path + ": cannot open file");
  size_t file_len = (size_t)f.tellg();
  f.seekg(0);
  std::vector<char> bytes(file_len);
  if (file_len && !f.read(bytes.data(), (std::streamsize)file_len))
    raise(PPOCR_ERR_READ_FILE, "read weights " + path + ": short read");
  if (file_len < 8) raise(PPOCR_ERR_SAFETENSORS, "decode safetensors: file shorter than its header length");
  uint64_t hlen = 0;
  memcpy(&hlen, bytes.data(), 8);
  if (hlen > file_len - 8) raise(PPOCR_ERR_SAFETENSORS, "decode safetensors: header exceeds file");
  std::string header(bytes.data() + 8, bytes.data() + 8 + hlen);
  const size_t base = 8 + hlen;
  const size_t data_len = file_len - base;

  SafeTensors st;
  Json j(header);
  j.expect('{');
  if (j.eat('}')) return st;
  do {
    std::string name = j.str();
    j.expect(':');
    if (name == "__metadata__") {
      j.skip();
      continue;
    }
    std::string dtype;
    std::vector<uint64_t> shape;
    uint64_t start = 0, end = 0;
    bool have_offsets = false;
    j.expect('{');
    if (!j.eat('}')) {
      do {
        std::string key = j.str();
        j.expect(':');
        if (key == "dtype") {
          dtype = j.str();
        } else if (key == "shape") {
          j.expect('[');
          if (!j.eat(']')) {
            do shape.push_back(j.uint());
            while (j.eat(','));
            j.expect(']');
          }
        } else if (key == "data_offsets") {
          j.expect('[');
          start = j.uint();
          j.expect(',');
          end = j.uint();
          j.expect(']');
          have_offsets = true;
        } else {
          j.skip();
        }
      } while (j.eat(','));
      j.expect('}');
    }
    if (!have_offsets) raise(PPOCR_ERR_SAFETENSORS, "decode safetensors: tensor " + name + " has no data_offsets");
    if (dtype != "F32") raise(PPOCR_ERR_UNSUPPORTED_DTYPE, "tensor \"" + name + "\" has dtype " + dtype + "; expected F32");
    HostTensor t;
    uint64_t count = 1;
    for (uint64_t d : shape) {
      if (d > INT32_MAX || (d && count > UINT64_MAX / 4 / d))
        raise(PPOCR_ERR_TENSOR_SIZE_OVERFLOW, "tensor \"" + name + "\" size overflows");
      count *= d;
      t.shape.push_back((int)d);
    }
    if (end < start || end > data_len)
      raise(PPOCR_ERR_INVALID_TENSOR_RANGE, "tensor \"" + name + "\" range " + std::to_string(start) + ".." +
                                                std::to_string(end) + " exceeds the data section of " +
                                                std::to_string(data_len) + " bytes");
    if (end - start != count * 4)
      raise(PPOCR_ERR_TENSOR_BYTE_LENGTH, "tensor \"" + name + "\" has " + std::to_string(end - start) +
                                              " bytes; expected " + std::to_string(count * 4));
    t.v.resize(count);
    if (count) memcpy(t.v.data(), bytes.data() + base + start, count * 4);
    st.tensors_.emplace(name, std::move(t));
  } while (j.eat(','));
  j.expect('}');
  return st;
}

HostTensor SafeTensors::get(const std::string& name, const std::vector<int>& shape) const {
  auto it = tensors_.find(name);
  if (it == tensors_.end()) raise(PPOCR_ERR_TENSOR_NOT_FOUND, "tensor \"" + name + "\" was not found");
  if (it->second.shape != shape) {
    auto fmt = [](const std::vector<int>& s) {
      std::string r = "[";
      for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
      return r + "]";
    };
    raise(PPOCR_ERR_SHAPE_MISMATCH,
          "tensor \"" + name + "\" has shape " + fmt(it->second.shape) + "; expected " + fmt(shape));
  }
  return it->second;
}

}  // namespace ppocr
