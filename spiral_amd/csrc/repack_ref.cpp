// Host repack of canonical GGUF weights into the reference's record layout:
// the quants_<fmt>_record_count / packed_bytes / repack entry points.
//
// Layouts (records ordered [weights_cols/8][weights_rows/record_rows]):
//   Q4_0 64 x 8, 288 B: fp16 d[2 blocks][8 cols], then per block 128 B of
//        signed nibbles (q - 8) & 15, byte row*4 + col/2, low nibble = even
//        column (src/quants/q4_0/layout.h:18-35, repack.h:48-107).
//   Q8_0 256 x 8, 2176 B: per block 4 tiles of 8 x 8 int8 (row-major), then
//        fp16 d[8 blocks][8 cols] (src/quants/q8_0/layout.h:15-36,
//        repack.h:53-83).
//   Q6_K 256 x 8, 1680 B: 4 chunks of 64 rows, each a 4-bit plane then a
//        2-bit plane over index row*8 + col; then sub-scales
//        [chunk][subgroup][col]; then fp16 d[8 cols]. Chunk c covers canonical
//        half c/2 and nibble c%2 (src/quants/q6_k/layout.h:17-42,
//        repack.h:46-108).
// Errors: 0 for a bad shape, short destination, short source stride or a
// null pointer (src/quants/q4_0/repack.h:33-41). A subnormal fp16 scale is
// stored as +0; one warning line per call (src/quants/common/repack.h:38-61),
// to stderr or to the callback set with quants_set_repack_warn (the
// reference routes it with its QUANTS_REPACK_WARN macro,
// src/quants/common/repack.h:9-14).
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "spiral_quants.h"

namespace {

// Where the warning line goes (quants_set_repack_warn); NULL: stderr.
std::mutex g_warn_mutex;
quants_warn_fn g_warn_fn = nullptr;
void* g_warn_user = nullptr;

void emit_warning(const char* line) {
  quants_warn_fn fn;
  void* user;
  {
    std::lock_guard<std::mutex> lock(g_warn_mutex);
    fn = g_warn_fn;
    user = g_warn_user;
  }
  if (fn != nullptr)
    fn(line, user);
  else
    fputs(line, stderr);
}

struct Geometry {
  const char* name;
  int record_rows;   // k extent of a record
  int record_bytes;
  int block_elems;   // canonical block
  int block_bytes;
};

constexpr Geometry kQ4_0{"Q4_0", 64, 288, 32, 18};
constexpr Geometry kQ8_0{"Q8_0", 256, 2176, 32, 34};
constexpr Geometry kQ6_K{"Q6_K", 256, 1680, 256, 210};

// Records of a rows x cols matrix, 0 for a shape the format cannot hold and
// for one whose record stream would not fit an int64 byte count (the
// reference's product is unchecked there).
int64_t record_count(const Geometry& g, int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0 || rows % g.record_rows != 0 || cols % 8 != 0) return 0;
  int64_t records = 0, bytes = 0;
  if (__builtin_mul_overflow(rows / g.record_rows, cols / 8, &records) ||
      __builtin_mul_overflow(records, static_cast<int64_t>(g.record_bytes), &bytes))
    return 0;
  return records;
}

struct Flags {
  bool subnormal = false;
  bool min_int8 = false;
  void report(const char* name) const {
    char line[128];
    if (subnormal && min_int8)
      snprintf(line, sizeof line, "quants: %s repack flushed subnormal fp16 scales to zero and found -128 int8 weights\n",
               name);
    else if (subnormal)
      snprintf(line, sizeof line, "quants: %s repack flushed subnormal fp16 scales to zero\n", name);
    else if (min_int8)
      snprintf(line, sizeof line, "quants: %s repack found -128 int8 weights\n", name);
    else
      return;
    emit_warning(line);
  }
};

inline void copy_scale(const uint8_t* src, uint8_t* dst, Flags& f) {
  const uint16_t bits = static_cast<uint16_t>(src[0] | (src[1] << 8));
  if ((bits & 0x7c00u) == 0 && (bits & 0x03ffu) != 0) {  // subnormal -> +0
    dst[0] = dst[1] = 0;
    f.subnormal = true;
  } else {
    dst[0] = src[0];
    dst[1] = src[1];
  }
}

// Fills one record from the 8 canonical columns whose blocks start at col[c].
void fill_q4_0(uint8_t* rec, const uint8_t* const col[8], int64_t block0, Flags& f) {
  memset(rec, 0, 288);
  for (int blk = 0; blk < 2; ++blk) {
    uint8_t* payload = rec + 32 + 128 * blk;
    for (int c = 0; c < 8; ++c) {
      const uint8_t* b = col[c] + (block0 + blk) * 18;
      copy_scale(b, rec + 16 * blk + 2 * c, f);
      const int shift = (c & 1) * 4;
      for (int j = 0; j < 16; ++j) {
        const uint8_t lo = static_cast<uint8_t>(((b[2 + j] & 15) - 8) & 15);
        const uint8_t hi = static_cast<uint8_t>(((b[2 + j] >> 4) - 8) & 15);
        payload[4 * j + c / 2] |= static_cast<uint8_t>(lo << shift);
        payload[4 * (j + 16) + c / 2] |= static_cast<uint8_t>(hi << shift);
      }
    }
  }
}

void fill_q8_0(uint8_t* rec, const uint8_t* const col[8], int64_t block0, Flags& f) {
  for (int blk = 0; blk < 8; ++blk) {
    for (int c = 0; c < 8; ++c) {
      const uint8_t* b = col[c] + (block0 + blk) * 34;
      copy_scale(b, rec + 2048 + 16 * blk + 2 * c, f);
      for (int j = 0; j < 32; ++j) {
        f.min_int8 |= b[2 + j] == 0x80u;
        rec[256 * blk + 8 * j + c] = b[2 + j];
      }
    }
  }
}

void fill_q6_k(uint8_t* rec, const uint8_t* const col[8], int64_t block0, Flags& f) {
  memset(rec, 0, 1536);
  for (int c = 0; c < 8; ++c) {
    const uint8_t* b = col[c] + block0 * 210;
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const uint8_t* sc = b + 192;
    copy_scale(b + 208, rec + 1664 + 2 * c, f);
    // Canonical element e = 128h + 32j + l; chunk = 2h + (j >> 1) holds it
    // at chunk row 32 * (j & 1) + l.
    for (int h = 0; h < 2; ++h) {
      for (int j = 0; j < 4; ++j) {
        const int chunk = 2 * h + (j >> 1);
        uint8_t* low = rec + 384 * chunk;
        uint8_t* high = low + 256;
        for (int s = 0; s < 2; ++s) {
          // sub-scale of rows 16s.. of group j&1 in this chunk
          rec[1536 + 32 * chunk + 8 * (2 * (j & 1) + s) + c] = sc[8 * h + 2 * j + s];
        }
        for (int l = 0; l < 32; ++l) {
          const int nib = (j >> 1) ? (ql[64 * h + 32 * (j & 1) + l] >> 4) : (ql[64 * h + 32 * (j & 1) + l] & 15);
          const int two = (qh[32 * h + l] >> (2 * j)) & 3;
          const int idx = (32 * (j & 1) + l) * 8 + c;
          low[idx >> 1] |= static_cast<uint8_t>(nib << (4 * (idx & 1)));
          high[idx >> 2] |= static_cast<uint8_t>(two << (2 * (idx & 3)));
        }
      }
    }
  }
}

int64_t repack(const Geometry& g, void (*fill)(uint8_t*, const uint8_t* const*, int64_t, Flags&),
               const uint8_t* src, int64_t stride, uint8_t* dst, int64_t capacity, int64_t rows, int64_t cols) {
  const int64_t records = record_count(g, rows, cols);
  const int64_t bytes = records * g.record_bytes;
  if (records == 0 || bytes > capacity || src == nullptr || dst == nullptr) return 0;
  if (stride < (rows / g.block_elems) * g.block_bytes) return 0;
  const int64_t row_records = rows / g.record_rows;
  const int64_t blocks_per_record = g.record_rows / g.block_elems;
  Flags flags;
  for (int64_t t = 0; t < cols / 8; ++t) {
    const uint8_t* col[8];
    for (int c = 0; c < 8; ++c) col[c] = src + (8 * t + c) * stride;
    for (int64_t r = 0; r < row_records; ++r)
      fill(dst + (t * row_records + r) * g.record_bytes, col, r * blocks_per_record, flags);
  }
  flags.report(g.name);
  return bytes;
}

}  // namespace

extern "C" {

int64_t quants_q4_0_record_count(int64_t r, int64_t c) { return record_count(kQ4_0, r, c); }
int64_t quants_q4_0_packed_bytes(int64_t r, int64_t c) { return record_count(kQ4_0, r, c) * kQ4_0.record_bytes; }
int64_t quants_q4_0_repack(const uint8_t* src, int64_t stride, uint8_t* dst, int64_t cap, int64_t r, int64_t c) {
  return repack(kQ4_0, fill_q4_0, src, stride, dst, cap, r, c);
}
int64_t quants_q8_0_record_count(int64_t r, int64_t c) { return record_count(kQ8_0, r, c); }
int64_t quants_q8_0_packed_bytes(int64_t r, int64_t c) { return record_count(kQ8_0, r, c) * kQ8_0.record_bytes; }
int64_t quants_q8_0_repack(const uint8_t* src, int64_t stride, uint8_t* dst, int64_t cap, int64_t r, int64_t c) {
  return repack(kQ8_0, fill_q8_0, src, stride, dst, cap, r, c);
}
int64_t quants_q6_k_record_count(int64_t r, int64_t c) { return record_count(kQ6_K, r, c); }
int64_t quants_q6_k_packed_bytes(int64_t r, int64_t c) { return record_count(kQ6_K, r, c) * kQ6_K.record_bytes; }
int64_t quants_q6_k_repack(const uint8_t* src, int64_t stride, uint8_t* dst, int64_t cap, int64_t r, int64_t c) {
  return repack(kQ6_K, fill_q6_k, src, stride, dst, cap, r, c);
}

void quants_set_repack_warn(quants_warn_fn fn, void* user) {
  std::lock_guard<std::mutex> lock(g_warn_mutex);
  g_warn_fn = fn;
  g_warn_user = user;
}

}  // extern "C"
