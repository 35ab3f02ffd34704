// t0mi_gptq.cpp — host side of the GPTQ container (GptqWeight,
// src/t0/quant_kernels.rs:177-294): header/section validation of the
// from_bytes byte layout, the gpu_buffer_size arithmetic, and the two facts the
// GPU conversion to the W4A16 layout depends on (zero points fit in 4 bits,
// scales survive bf16 rounding).
#include <string.h>

#include "t0mi_internal.h"

using namespace t0mi;

namespace {

uint32_t le32(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

}  // namespace

// GptqWeight::from_bytes (quant_kernels.rs:242-286).  Where the reference
// asserts (header < 12 bytes, truncated data, length mismatch), divides by a
// zero group size or drops the last nibble of an odd element count, this
// returns T0MI_ERR_INVALID with the reason.
extern "C" int t0mi_gptq_parse(const void* raw, size_t len, t0mi_gptq_info* out) {
  if (!raw || !out) return set_error(T0MI_ERR_INVALID, "null pointer");
  const uint8_t* b = (const uint8_t*)raw;
  if (len < 12) return set_error(T0MI_ERR_INVALID, "GPTQ data too short (need at least 12 bytes header)");
  t0mi_gptq_info info;
  memset(&info, 0, sizeof info);
  info.rows = le32(b);
  info.cols = le32(b + 4);
  info.group_size = le32(b + 8);
  if (info.group_size == 0) return set_error(T0MI_ERR_INVALID, "GPTQ group_size is 0");
  // Two INT4 values per byte: an odd element count cannot be packed (the
  // reference's rows * cols / 2 would silently drop the last nibble).
  if (((uint64_t)info.rows * info.cols) & 1)
    return set_error(T0MI_ERR_INVALID, "GPTQ rows * cols = %llu is odd (two INT4 values per byte)",
                     (unsigned long long)info.rows * info.cols);
  info.n_groups = info.cols / info.group_size;
  const uint64_t n_params = (uint64_t)info.n_groups * info.rows;  // < 2^64: both factors < 2^32
  info.packed_offset = 12;
  info.packed_bytes = (uint64_t)info.rows * info.cols / 2;
  // The section sizes can pass 2^64 bytes for header values near 2^32 (n_params * 8
  // wraps), so the length check is made in 128-bit arithmetic before any offset
  // is formed: a wrapped total would let the scan below read past the buffer.
  const unsigned __int128 total =
      (unsigned __int128)info.packed_offset + info.packed_bytes + (unsigned __int128)n_params * 8u;
  if (total > (unsigned __int128)len) {
    if (total >> 64)
      return set_error(T0MI_ERR_INVALID, "GPTQ data truncated: the header (rows %u, cols %u, group %u) needs "
                       "more than 2^64 bytes, got %zu", info.rows, info.cols, info.group_size, len);
    return set_error(T0MI_ERR_INVALID, "GPTQ data truncated: need %llu bytes, got %zu",
                     (unsigned long long)total, len);
  }
  info.scales_offset = info.packed_offset + info.packed_bytes;
  info.zeros_offset = info.scales_offset + n_params * 4;
  info.total_bytes = info.zeros_offset + n_params * 4;
  info.zeros_in_range = 1;
  info.scales_bf16_exact = 1;
  for (uint64_t i = 0; i < n_params; ++i) {
    const uint32_t sbits = le32(b + info.scales_offset + 4 * i);
    if (sbits & 0xFFFFu) info.scales_bf16_exact = 0;
    const int32_t z = (int32_t)le32(b + info.zeros_offset + 4 * i);
    if (z < 0 || z > 15) info.zeros_in_range = 0;
  }
  *out = info;
  return T0MI_OK;
}

// GptqWeight::gpu_buffer_size (quant_kernels.rs:289-293).
extern "C" uint64_t t0mi_gptq_gpu_buffer_size(const t0mi_gptq_info* info) {
  if (!info) return 0;
  const uint64_t n_params = (uint64_t)info->n_groups * info->rows;
  return info->packed_bytes + n_params * 4 + n_params * 4;
}
