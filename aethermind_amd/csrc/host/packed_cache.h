// On-disk cache of a model's repacked device weights (SavePackedCache /
// LoadPackedCache of model_weight_packing_strategy.md:390-394, design-only in the
// reference).  The file is the model's weight slab exactly as the repack kernels left
// it in HBM, behind a 256-byte header, so a load is a sequential read + DMA with no
// conversion or quantization.
//
// Layout (little-endian):
//   [0, 256)  header
//       0   char[8]   magic "AMPKGFX1"
//       8   u32       file format version (kVersion)
//       12  u32       header bytes (256)
//       16  u64       payload bytes
//       24  u64       payload checksum (PayloadHasher)
//       32  char[16]  device architecture the kernels read the payload with ("gfx950")
//       48  u32       slab layout version (kLayoutVersion: the order, alignment and
//                     device formats of the weights inside the payload)
//       52  i32 x 7   num_layers, hidden, num_q_heads, num_kv_heads, head_dim, ffn, vocab
//       80  f32       rms_eps
//       84  u32       zero
//       88  f64       rope_theta
//       96  i32 x 3   act_dtype, weight_format, group_size
//       108 .. 248    zero
//       248 u64       header checksum (PayloadHasher over bytes [0, 248))
//   [256, 256 + payload)  the weight slab (embedding, per-layer norms and linear
//                         weights, final norm, lm_head; 256-byte aligned pieces)
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

#include "am_core.h"
#include "am_runtime.h"

namespace aethermind::packed {

constexpr char kMagic[8] = {'A', 'M', 'P', 'K', 'G', 'F', 'X', '1'};
constexpr uint32_t kVersion = 1;
constexpr uint32_t kHeaderBytes = 256;
constexpr uint32_t kLayoutVersion = 1;
constexpr const char* kArch = "gfx950";

// 64-bit corruption check over a byte stream fed in 32-byte multiples (a final short
// piece is zero-padded): four independent multiply-rotate lanes, folded with the
// length at the end.  Not a cryptographic hash.
class PayloadHasher {
 public:
  void Update(const void* data, size_t n);
  uint64_t Finish() const;

 private:
  uint64_t h_[4] = {0x243F6A8885A308D3ull, 0x13198A2E03707344ull, 0xA4093822299F31D0ull, 0x082EFA98EC4E6C89ull};
  uint64_t len_ = 0;
};

uint64_t Checksum(const void* data, size_t n);

struct Header {
  uint64_t payload_bytes = 0;
  uint64_t payload_checksum = 0;
  am_model_config cfg{};  // max_tokens / max_prefill_chunk are not part of the file
};

// Serialises h into out[kHeaderBytes] (header checksum included).
void EncodeHeader(const Header& h, uint8_t* out);
// Parses and checks a header: magic, version, header size and checksum, architecture,
// layout version and the model config (positive dimensions, divisibility, known dtypes).
StatusOr<Header> DecodeHeader(const uint8_t* in, size_t n);
// Reads the header of a cache file and checks that the file holds the whole payload.
StatusOr<Header> Inspect(const std::string& path);

}  // namespace aethermind::packed
