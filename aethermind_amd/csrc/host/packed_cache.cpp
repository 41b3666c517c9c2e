#include "packed_cache.h"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstring>

namespace aethermind::packed {
namespace {

constexpr uint64_t kMul = 0x9E3779B97F4A7C15ull;

inline uint64_t Rotl(uint64_t v, int r) { return (v << r) | (v >> (64 - r)); }
inline uint64_t Mix(uint64_t h, uint64_t w) { return Rotl((h ^ w) * kMul, 29); }

template <class T>
void Put(uint8_t* out, size_t off, T v) {
  std::memcpy(out + off, &v, sizeof(T));
}
template <class T>
T Get(const uint8_t* in, size_t off) {
  T v;
  std::memcpy(&v, in + off, sizeof(T));
  return v;
}

constexpr size_t kOffMagic = 0, kOffVersion = 8, kOffHeaderBytes = 12, kOffPayload = 16, kOffPayloadSum = 24,
                 kOffArch = 32, kOffLayout = 48, kOffDims = 52, kOffEps = 80, kOffTheta = 88, kOffFormats = 96,
                 kOffHeaderSum = 248;

Status CheckConfig(const am_model_config& c) {
  if (c.num_layers <= 0 || c.hidden <= 0 || c.num_q_heads <= 0 || c.num_kv_heads <= 0 || c.head_dim <= 0 ||
      c.ffn <= 0 || c.vocab <= 0)
    return Status::InvalidArgument("packed cache: model dimensions must be positive");
  if (c.num_q_heads % c.num_kv_heads != 0)
    return Status::InvalidArgument("packed cache: num_attention_heads must be divisible by num_key_value_heads");
  if (!(c.rms_eps > 0.0f) || !(c.rope_theta > 0.0) || !std::isfinite(c.rope_theta))
    return Status::InvalidArgument("packed cache: rms_eps and rope_theta must be positive");
  if (c.act_dtype != AM_DT_F32 && c.act_dtype != AM_DT_BF16)
    return Status::InvalidArgument("packed cache: unknown activation dtype");
  if (c.weight_format < AM_WF_F32 || c.weight_format > AM_WF_INT4)
    return Status::InvalidArgument("packed cache: unknown weight format");
  if (c.weight_format == AM_WF_INT4 && c.group_size <= 0)
    return Status::InvalidArgument("packed cache: INT4 weights need a positive group size");
  return Status::Ok();
}

}  // namespace

void PayloadHasher::Update(const void* data, size_t n) {
  const uint8_t* p = static_cast<const uint8_t*>(data);
  len_ += n;
  size_t i = 0;
  for (; i + 32 <= n; i += 32) {
    h_[0] = Mix(h_[0], Get<uint64_t>(p, i));
    h_[1] = Mix(h_[1], Get<uint64_t>(p, i + 8));
    h_[2] = Mix(h_[2], Get<uint64_t>(p, i + 16));
    h_[3] = Mix(h_[3], Get<uint64_t>(p, i + 24));
  }
  if (i < n) {  // zero-padded tail: only the last piece of a stream may be short
    uint8_t tail[32] = {0};
    std::memcpy(tail, p + i, n - i);
    for (int l = 0; l < 4; ++l) h_[l] = Mix(h_[l], Get<uint64_t>(tail, 8 * l));
  }
}

uint64_t PayloadHasher::Finish() const {
  uint64_t h = len_ * kMul;
  for (int l = 0; l < 4; ++l) h = Mix(h, h_[l]);
  return h ^ (h >> 31);
}

uint64_t Checksum(const void* data, size_t n) {
  PayloadHasher h;
  h.Update(data, n);
  return h.Finish();
}

void EncodeHeader(const Header& h, uint8_t* out) {
  std::memset(out, 0, kHeaderBytes);
  std::memcpy(out + kOffMagic, kMagic, sizeof(kMagic));
  Put<uint32_t>(out, kOffVersion, kVersion);
  Put<uint32_t>(out, kOffHeaderBytes, kHeaderBytes);
  Put<uint64_t>(out, kOffPayload, h.payload_bytes);
  Put<uint64_t>(out, kOffPayloadSum, h.payload_checksum);
  std::strncpy(reinterpret_cast<char*>(out + kOffArch), kArch, 15);
  Put<uint32_t>(out, kOffLayout, kLayoutVersion);
  const am_model_config& c = h.cfg;
  const int32_t dims[7] = {c.num_layers, c.hidden, c.num_q_heads, c.num_kv_heads, c.head_dim, c.ffn, c.vocab};
  for (int i = 0; i < 7; ++i) Put<int32_t>(out, kOffDims + 4 * i, dims[i]);
  Put<float>(out, kOffEps, c.rms_eps);
  Put<double>(out, kOffTheta, c.rope_theta);
  Put<int32_t>(out, kOffFormats, c.act_dtype);
  Put<int32_t>(out, kOffFormats + 4, c.weight_format);
  Put<int32_t>(out, kOffFormats + 8, c.group_size);
  Put<uint64_t>(out, kOffHeaderSum, Checksum(out, kOffHeaderSum));
}

StatusOr<Header> DecodeHeader(const uint8_t* in, size_t n) {
  if (n < kHeaderBytes) return Status::DataLoss("packed cache: file shorter than its header");
  if (std::memcmp(in + kOffMagic, kMagic, sizeof(kMagic)) != 0)
    return Status::InvalidArgument("packed cache: not a packed weight cache (bad magic)");
  if (Get<uint32_t>(in, kOffVersion) != kVersion || Get<uint32_t>(in, kOffHeaderBytes) != kHeaderBytes)
    return Status::FailedPrecondition("packed cache: unsupported file format version");
  if (Get<uint64_t>(in, kOffHeaderSum) != Checksum(in, kOffHeaderSum))
    return Status::DataLoss("packed cache: header checksum mismatch");
  char arch[17] = {0};
  std::memcpy(arch, in + kOffArch, 16);
  if (std::strcmp(arch, kArch) != 0)
    return Status::FailedPrecondition(std::string("packed cache: written for ") + arch + ", this library runs " + kArch);
  if (Get<uint32_t>(in, kOffLayout) != kLayoutVersion)
    return Status::FailedPrecondition("packed cache: written with another weight layout version; repack from the checkpoint");
  Header h;
  h.payload_bytes = Get<uint64_t>(in, kOffPayload);
  h.payload_checksum = Get<uint64_t>(in, kOffPayloadSum);
  am_model_config& c = h.cfg;
  c.num_layers = Get<int32_t>(in, kOffDims);
  c.hidden = Get<int32_t>(in, kOffDims + 4);
  c.num_q_heads = Get<int32_t>(in, kOffDims + 8);
  c.num_kv_heads = Get<int32_t>(in, kOffDims + 12);
  c.head_dim = Get<int32_t>(in, kOffDims + 16);
  c.ffn = Get<int32_t>(in, kOffDims + 20);
  c.vocab = Get<int32_t>(in, kOffDims + 24);
  c.rms_eps = Get<float>(in, kOffEps);
  c.rope_theta = Get<double>(in, kOffTheta);
  c.act_dtype = Get<int32_t>(in, kOffFormats);
  c.weight_format = Get<int32_t>(in, kOffFormats + 4);
  c.group_size = Get<int32_t>(in, kOffFormats + 8);
  AM_RETURN_IF_ERROR(CheckConfig(c));
  if (h.payload_bytes == 0 || h.payload_bytes % 256 != 0)
    return Status::DataLoss("packed cache: payload size is not a whole number of 256-byte pieces");
  return h;
}

StatusOr<Header> Inspect(const std::string& path) {
  const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return Status::NotFound("packed cache: cannot open " + path + ": " + std::strerror(errno));
  uint8_t buf[kHeaderBytes];
  const ssize_t got = ::pread(fd, buf, kHeaderBytes, 0);
  struct stat st {};
  const int sr = ::fstat(fd, &st);
  ::close(fd);
  if (got < 0 || sr != 0) return Status::Internal("packed cache: cannot read " + path);
  auto h = DecodeHeader(buf, static_cast<size_t>(got));
  if (!h.ok()) return h.status();
  if (static_cast<uint64_t>(st.st_size) != kHeaderBytes + h.value().payload_bytes)
    return Status::DataLoss("packed cache: file size does not match the header's payload size (truncated or padded)");
  return h;
}

}  // namespace aethermind::packed
