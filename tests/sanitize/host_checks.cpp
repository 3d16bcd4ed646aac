// Host-side checks of libspiral_quants' C/C++ code under AddressSanitizer and
// UndefinedBehaviorSanitizer, with no GPU: built by tests/sanitize/Makefile
// (host code instrumented, device code untouched) and run by
// tests/test_sanitize.py.
//
// What runs:
//  - the reference-layout host repack (quants_<fmt>_*) at valid and invalid
//    shapes, padded column strides, exact and short capacities and null
//    pointers, byte-compared with the oracle's restatement, plus the warning
//    route;
//  - the oracle's dequant / GET_ROWS / record unpack / matmul functions and
//    the CPU baseline at ragged shapes with padded strides;
//  - every argument check of the device entry points and of the ggml
//    surface that returns before device work (null, misaligned, negative,
//    overflowing sizes), and the size queries at extreme arguments;
//  - the llama.cpp shim's tensor conversion, restated from INTEGRATION.md
//    over a minimal ggml_tensor, on storage filled with garbage first: a row
//    view and a whole-expert view of a weight through spiral_supports_op
//    (which reads view_src before any buffer check) and the size query.
// Any sanitizer report aborts the program (-fno-sanitize-recover=all); a
// failed expectation prints the case and makes the exit status nonzero.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <vector>

#include "spiral_ggml.h"
#include "spiral_quants.h"

extern "C" {
#include "quants_oracle.h"
int cb_gemv_q8_0(const uint8_t* raw, int64_t n_rows, int64_t k, const uint16_t* x, float* y, int threads);
int cb_dequant_q4_0(const uint8_t* raw, int64_t n_rows, int64_t k, uint16_t* out, int threads);
int cb_gemm_q4_0(const uint8_t* raw, int64_t n_rows, int64_t k, const uint16_t* x, int64_t m, float* y,
                 int threads);
}

namespace {

int g_failures = 0;

#define EXPECT(cond, ...)                                   \
  do {                                                      \
    if (!(cond)) {                                          \
      ++g_failures;                                         \
      std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
      std::fprintf(stderr, __VA_ARGS__);                    \
      std::fprintf(stderr, "\n");                           \
    }                                                       \
  } while (0)

uint64_t g_rng = 0x9E3779B97F4A7C15ull;
uint32_t rnd() {
  g_rng ^= g_rng << 13;
  g_rng ^= g_rng >> 7;
  g_rng ^= g_rng << 17;
  return static_cast<uint32_t>(g_rng >> 16);
}

// Canonical GGUF bytes with normal fp16 scales at every scale field; a few
// scales are made subnormal when `subnormal` is set.
std::vector<uint8_t> random_blocks(int type, int64_t n_blocks, bool subnormal) {
  const int bb = oq_block_bytes(type);
  std::vector<uint8_t> v(static_cast<size_t>(n_blocks * bb));
  for (auto& b : v) b = static_cast<uint8_t>(rnd());
  for (int64_t i = 0; i < n_blocks; ++i) {
    uint8_t* blk = v.data() + i * bb;
    uint16_t d = static_cast<uint16_t>(0x2000 + (rnd() & 0x0FFF));  // normal, modest
    if (subnormal && i % 7 == 3) d = static_cast<uint16_t>(rnd() & 0x03FF);
    // fp16 scale positions: Q4_0/Q8_0/IQ4_NL/IQ4_XS and the K-quants lead with d
    // (K-quants: d then dmin); Q6_K ends with d.
    size_t at = type == OQ_Q6_K ? static_cast<size_t>(bb - 2) : 0;
    blk[at] = static_cast<uint8_t>(d);
    blk[at + 1] = static_cast<uint8_t>(d >> 8);
    if (type == OQ_Q4_K || type == OQ_Q5_K) {
      blk[2] = static_cast<uint8_t>(d);
      blk[3] = static_cast<uint8_t>(d >> 8);
    }
  }
  return v;
}

std::vector<uint16_t> random_bf16(int64_t n) {
  std::vector<uint16_t> v(static_cast<size_t>(n));
  for (auto& x : v) x = oq_bf16_rne((static_cast<float>(rnd() % 2001) - 1000.0f) / 512.0f);
  return v;
}

// ---- host repack against the oracle -----------------------------------------

struct RepackFns {
  int type;
  const char* name;
  int64_t (*count)(int64_t, int64_t);
  int64_t (*bytes)(int64_t, int64_t);
  int64_t (*repack)(const uint8_t*, int64_t, uint8_t*, int64_t, int64_t, int64_t);
};

int g_warn_calls = 0;
void count_warn(const char*, void* user) {
  if (user == &g_warn_calls) ++g_warn_calls;
}

void check_repack() {
  const RepackFns fns[] = {
      {OQ_Q4_0, "q4_0", quants_q4_0_record_count, quants_q4_0_packed_bytes, quants_q4_0_repack},
      {OQ_Q8_0, "q8_0", quants_q8_0_record_count, quants_q8_0_packed_bytes, quants_q8_0_repack},
      {OQ_Q6_K, "q6_k", quants_q6_k_record_count, quants_q6_k_packed_bytes, quants_q6_k_repack},
  };
  const int64_t rows_list[] = {0, 32, 64, 96, 128, 256, 512, 768, -64};
  const int64_t cols_list[] = {0, 4, 8, 12, 16, 24, -8};
  quants_set_repack_warn(count_warn, &g_warn_calls);
  for (const RepackFns& f : fns) {
    const int be = oq_block_elems(f.type), bb = oq_block_bytes(f.type);
    for (int64_t rows : rows_list)
      for (int64_t cols : cols_list) {
        const int64_t want_count = oq_ref_record_count(f.type, rows, cols);
        const int64_t want_bytes = oq_ref_packed_bytes(f.type, rows, cols);
        EXPECT(f.count(rows, cols) == want_count, "%s record_count(%lld, %lld)", f.name, (long long)rows,
               (long long)cols);
        EXPECT(f.bytes(rows, cols) == want_bytes, "%s packed_bytes(%lld, %lld)", f.name, (long long)rows,
               (long long)cols);
        if (want_bytes <= 0) continue;
        for (int64_t pad : {int64_t(0), int64_t(2), int64_t(16), int64_t(37)}) {
          const int64_t stride = rows / be * bb + pad;
          std::vector<uint8_t> src = random_blocks(f.type, cols * (stride / bb + 1), pad == 16);
          src.resize(static_cast<size_t>(cols * stride));
          // Re-normalize the blocks of each column at the strided positions.
          for (int64_t c = 0; c < cols; ++c) {
            std::vector<uint8_t> col = random_blocks(f.type, rows / be, pad == 16);
            std::memcpy(src.data() + c * stride, col.data(), col.size());
          }
          std::vector<uint8_t> want(static_cast<size_t>(want_bytes)), got(static_cast<size_t>(want_bytes) + 64, 0xA5);
          int warnings = 0;
          const int64_t w = oq_ref_repack(f.type, src.data(), stride, want.data(), want_bytes, rows, cols, &warnings);
          EXPECT(w == want_bytes, "oracle %s repack", f.name);
          g_warn_calls = 0;
          const int64_t r = f.repack(src.data(), stride, got.data(), want_bytes, rows, cols);
          EXPECT(r == want_bytes, "%s repack(%lld x %lld, stride %lld) = %lld", f.name, (long long)rows,
                 (long long)cols, (long long)stride, (long long)r);
          EXPECT(std::memcmp(got.data(), want.data(), static_cast<size_t>(want_bytes)) == 0, "%s repack bytes",
                 f.name);
          EXPECT(got[static_cast<size_t>(want_bytes)] == 0xA5, "%s repack wrote past its capacity", f.name);
          EXPECT(g_warn_calls == (warnings != 0 ? 1 : 0), "%s warning count %d (oracle flags %d)", f.name,
                 g_warn_calls, warnings);
          // Short capacity, null pointers, bad strides: 0 and nothing written.
          std::vector<uint8_t> small(static_cast<size_t>(want_bytes - 1), 0x5A);
          EXPECT(f.repack(src.data(), stride, small.data(), want_bytes - 1, rows, cols) == 0, "%s short capacity",
                 f.name);
          EXPECT(f.repack(nullptr, stride, got.data(), want_bytes, rows, cols) == 0, "%s null src", f.name);
          EXPECT(f.repack(src.data(), stride, nullptr, want_bytes, rows, cols) == 0, "%s null dst", f.name);
          EXPECT(f.repack(src.data(), -stride, got.data(), want_bytes, rows, cols) == 0, "%s negative stride",
                 f.name);
          EXPECT(f.repack(src.data(), rows / be * bb - 1, got.data(), want_bytes, rows, cols) == 0,
                 "%s stride below a column", f.name);
        }
      }
    const int64_t big = std::numeric_limits<int64_t>::max();
    EXPECT(f.count(big, big) == oq_ref_record_count(f.type, big, big), "%s record_count(max, max)", f.name);
    EXPECT(f.bytes(big, 8) == oq_ref_packed_bytes(f.type, big, 8), "%s packed_bytes(max, 8)", f.name);
    EXPECT(f.bytes(256, big - 7) == oq_ref_packed_bytes(f.type, 256, big - 7), "%s packed_bytes(256, max)", f.name);
  }
  quants_set_repack_warn(nullptr, nullptr);
}

// ---- oracle and CPU baseline -------------------------------------------------

void check_oracle() {
  const int types[] = {OQ_Q4_0, OQ_Q8_0, OQ_Q6_K, OQ_Q4_K, OQ_Q5_K, OQ_IQ4_NL, OQ_IQ4_XS};
  for (int type : types) {
    const int be = oq_block_elems(type), bb = oq_block_bytes(type);
    const int64_t n = 13, k = 3 * be, stride = k / be * bb + 6, ld_out = k + 5;
    std::vector<uint8_t> src(static_cast<size_t>(n * stride));
    for (int64_t r = 0; r < n; ++r) {
      std::vector<uint8_t> row = random_blocks(type, k / be, true);
      std::memcpy(src.data() + r * stride, row.data(), row.size());
    }
    std::vector<uint16_t> out(static_cast<size_t>(n * ld_out), 0x7777);
    EXPECT(oq_dequant(type, src.data(), stride, n, k, out.data(), ld_out) == 0, "oq_dequant type %d", type);
    EXPECT(out[static_cast<size_t>(k)] == 0x7777, "oq_dequant wrote into row padding (type %d)", type);
    EXPECT(oq_dequant(type, src.data(), stride, n, k + 1, out.data(), ld_out) != 0, "oq_dequant bad k (type %d)",
           type);
    std::vector<double> wd(static_cast<size_t>(n * k));
    EXPECT(oq_dequant_f64(type, src.data(), stride, n, k, wd.data(), k) == 0, "oq_dequant_f64 type %d", type);
    const int32_t ids[] = {0, 12, 5, 12, 3, 7}, bad[] = {0, -1}, past[] = {13};
    std::vector<uint16_t> rows(static_cast<size_t>(6 * k));
    EXPECT(oq_get_rows(type, src.data(), stride, n, k, bad, 2, rows.data(), k) != 0, "oq_get_rows id -1");
    EXPECT(oq_get_rows(type, src.data(), stride, n, k, past, 1, rows.data(), k) != 0, "oq_get_rows id n");
    EXPECT(oq_get_rows(type, src.data(), stride, n, k, ids, 6, rows.data(), k) == 0, "oq_get_rows type %d", type);
    EXPECT(std::memcmp(rows.data() + k, out.data() + 12 * ld_out, static_cast<size_t>(k) * 2) == 0,
           "oq_get_rows row 12 (type %d)", type);
    const int64_t m = 3;
    std::vector<uint16_t> x = random_bf16(m * (k + 8));
    std::vector<float> y32(static_cast<size_t>(m * (n + 2)));
    EXPECT(oq_quant_matmul_f32(type, src.data(), stride, n, k, x.data(), k + 8, m, y32.data(), n + 2, 3) == 0,
           "oq_quant_matmul_f32 type %d", type);
    std::vector<double> y64(static_cast<size_t>(m * n));
    oq_matmul_f64(out.data(), ld_out, n, k, x.data(), k + 8, m, y64.data(), n);
    std::vector<float> yf(static_cast<size_t>(m * n));
    oq_matmul_f32(out.data(), ld_out, n, k, x.data(), k + 8, m, yf.data(), n);
    for (int64_t i = 0; i < m * n; ++i) {
      const double ref = y64[static_cast<size_t>(i)];
      const double got = y32[static_cast<size_t>(i / n * (n + 2) + i % n)];
      EXPECT(got - ref < 1e-2 * (1.0 + (ref < 0 ? -ref : ref)) && ref - got < 1e-2 * (1.0 + (ref < 0 ? -ref : ref)),
             "oq_quant_matmul_f32 vs f64 (type %d, %lld)", type, (long long)i);
    }
    std::vector<double> ye(static_cast<size_t>(m * n));
    oq_matmul_f64_exact(wd.data(), k, n, k, x.data(), k + 8, m, ye.data(), n);
  }
  // Record unpack over a repacked matrix, all three record formats.
  for (int type : {OQ_Q4_0, OQ_Q8_0, OQ_Q6_K}) {
    const int be = oq_block_elems(type), bb = oq_block_bytes(type);
    const int64_t rows = 512, cols = 16, stride = rows / be * bb;
    std::vector<uint8_t> src = random_blocks(type, cols * rows / be, false);
    const int64_t pb = oq_ref_packed_bytes(type, rows, cols);
    std::vector<uint8_t> rec(static_cast<size_t>(pb));
    int warnings = 0;
    EXPECT(oq_ref_repack(type, src.data(), stride, rec.data(), pb, rows, cols, &warnings) == pb, "repack %d", type);
    std::vector<uint16_t> un(static_cast<size_t>(rows * cols));
    EXPECT(oq_ref_unpack(type, rec.data(), rows, cols, un.data()) == 0, "oq_ref_unpack type %d", type);
  }
  int64_t signed_zero = 0;
  EXPECT(oq_check_q6_k(257, &signed_zero) == 0, "oq_check_q6_k");
  EXPECT(oq_check_split_identity() == 0, "oq_check_split_identity");

  // CPU baseline: ragged row counts (the GEMM's 8-row tile tail), 1 and 3 threads.
  for (int threads : {1, 3}) {
    const int64_t n = 21, k = 96, m = 2;
    std::vector<uint8_t> q4 = random_blocks(OQ_Q4_0, n * k / 32, false);
    std::vector<uint8_t> q8 = random_blocks(OQ_Q8_0, n * k / 32, false);
    std::vector<uint16_t> x = random_bf16(m * k);
    std::vector<float> y(static_cast<size_t>(m * n)), ref(static_cast<size_t>(m * n));
    EXPECT(cb_gemv_q8_0(q8.data(), n, k, x.data(), y.data(), threads) == 0, "cb_gemv_q8_0");
    oq_quant_matmul_f32(OQ_Q8_0, q8.data(), k / 32 * 34, n, k, x.data(), k, 1, ref.data(), n, 1);
    for (int64_t i = 0; i < n; ++i) EXPECT(y[i] - ref[i] < 1e-2f && ref[i] - y[i] < 1e-2f, "cb_gemv_q8_0 row %lld", (long long)i);
    std::vector<uint16_t> dq(static_cast<size_t>(n * k)), dq_ref(static_cast<size_t>(n * k));
    EXPECT(cb_dequant_q4_0(q4.data(), n, k, dq.data(), threads) == 0, "cb_dequant_q4_0");
    oq_dequant(OQ_Q4_0, q4.data(), k / 32 * 18, n, k, dq_ref.data(), k);
    EXPECT(dq == dq_ref, "cb_dequant_q4_0 bits");
    EXPECT(cb_gemm_q4_0(q4.data(), n, k, x.data(), m, y.data(), threads) == 0, "cb_gemm_q4_0");
    EXPECT(cb_gemm_q4_0(q4.data(), n, k + 1, x.data(), m, y.data(), threads) != 0, "cb_gemm_q4_0 bad k");
  }
}

// ---- argument checks of the device entry points and the ggml surface ------------

void check_validation() {
  const int64_t big = std::numeric_limits<int64_t>::max();
  const int types[] = {SPIRAL_TYPE_Q4_0, SPIRAL_TYPE_Q8_0, SPIRAL_TYPE_Q6_K, SPIRAL_TYPE_Q4_K,
                       SPIRAL_TYPE_Q5_K, SPIRAL_TYPE_IQ4_NL, SPIRAL_TYPE_IQ4_XS};
  for (int t : types) {
    for (int64_t k : {int64_t(0), int64_t(-256), int64_t(256), int64_t(4096), big, big - 255, big / 2}) {
      const int64_t rb = spiral_row_bytes(t, k);
      EXPECT(rb >= 0, "spiral_row_bytes(%d, %lld) < 0", t, (long long)k);
      for (int64_t n : {int64_t(1), int64_t(-1), big, int64_t(1) << 40})
        EXPECT(spiral_tensor_bytes(t, n, k) >= 0, "spiral_tensor_bytes(%d, %lld, %lld) < 0", t, (long long)n,
               (long long)k);
    }
    for (int64_t m : {int64_t(1), int64_t(4), int64_t(512), big})
      for (int64_t k : {int64_t(256), int64_t(4096), big - 255})
        EXPECT(spiral_mul_mat_workspace_bytes(t, 4096, k, m) >= 0, "workspace(%d, m=%lld, k=%lld)", t,
               (long long)m, (long long)k);
  }
  EXPECT(spiral_row_bytes(99, 256) == 0, "unknown type row bytes");
  EXPECT(spiral_mul_mat_id_workspace_bytes(big, big, big) >= 0, "mul_mat_id workspace at max");
  EXPECT(spiral_mul_mat_id_workspace_bytes(128, big / 2, 8) >= 0, "mul_mat_id workspace n_tokens*top_k overflow");

  alignas(16) static uint8_t wbuf[4096];
  alignas(16) static uint16_t xbuf[4096];
  alignas(16) static float ybuf[1024];
  alignas(16) static int32_t ids[64];
  const int q = SPIRAL_TYPE_Q4_0;
  EXPECT(spiral_mul_mat(99, wbuf, 8, 32, xbuf, 32, 1, ybuf, SPIRAL_TYPE_F32, 8, nullptr, 0, nullptr) ==
             SPIRAL_ERR_TYPE, "mul_mat type");
  EXPECT(spiral_mul_mat(q, nullptr, 8, 32, xbuf, 32, 1, ybuf, SPIRAL_TYPE_F32, 8, nullptr, 0, nullptr) ==
             SPIRAL_ERR_NULL, "mul_mat null");
  EXPECT(spiral_mul_mat(q, wbuf, 8, 33, xbuf, 40, 1, ybuf, SPIRAL_TYPE_F32, 8, nullptr, 0, nullptr) ==
             SPIRAL_ERR_SHAPE, "mul_mat k");
  EXPECT(spiral_mul_mat(q, wbuf + 2, 8, 32, xbuf, 32, 1, ybuf, SPIRAL_TYPE_F32, 8, nullptr, 0, nullptr) ==
             SPIRAL_ERR_ALIGN, "mul_mat align");
  EXPECT(spiral_mul_mat(q, wbuf, big, big - 31, xbuf, big, big, ybuf, SPIRAL_TYPE_F32, big, nullptr, 0, nullptr) !=
             SPIRAL_OK, "mul_mat at max sizes");
  EXPECT(spiral_mul_mat(q, wbuf, 8, 32, xbuf, 32, 512, ybuf, SPIRAL_TYPE_F32, 8, nullptr, 0, nullptr) ==
             SPIRAL_ERR_NULL, "mul_mat GEMM without workspace");
  EXPECT(spiral_dequant_bf16(q, wbuf, 8, 33, xbuf, 33, nullptr) != SPIRAL_OK, "dequant k");
  EXPECT(spiral_dequant_bf16(q, wbuf, big, big - 31, xbuf, big, nullptr) != SPIRAL_OK, "dequant at max");
  EXPECT(spiral_get_rows(q, wbuf, 8, 32, ids, -1, ybuf, SPIRAL_TYPE_F32, 32, nullptr) != SPIRAL_OK, "get_rows n");
  EXPECT(spiral_to_planar(q, wbuf, 18, big, 32, wbuf, nullptr) != SPIRAL_OK, "to_planar at max");
  EXPECT(spiral_from_planar(q, wbuf, 8, 32, wbuf, 1, nullptr) != SPIRAL_OK, "from_planar stride");
  for (int64_t nt : {int64_t(-1), big / 2, big}) {
    EXPECT(spiral_mul_mat_id(q, wbuf, 144, 4, 8, 32, xbuf, 1, ids, nt, 8, ybuf, SPIRAL_TYPE_F32, wbuf, 4096,
                             nullptr) != SPIRAL_OK, "mul_mat_id n_tokens %lld", (long long)nt);
    EXPECT(spiral_mul_mat_id_noalloc(q, wbuf, 144, 4, 8, 32, xbuf, 1, ids, nt, 8, ybuf, SPIRAL_TYPE_F32,
                                     nullptr) != SPIRAL_OK, "mul_mat_id_noalloc n_tokens %lld", (long long)nt);
  }
  EXPECT(spiral_mul_mat_id(q, wbuf, big, big, big, big - 31, xbuf, 1, ids, 4, big, ybuf, SPIRAL_TYPE_F32, wbuf,
                           big, nullptr) != SPIRAL_OK, "mul_mat_id at max");
  EXPECT(spiral_mul_mat_id_glu(q, wbuf, 144, 4, 7, 32, xbuf, 1, ids, 4, 2, SPIRAL_GLU_SWIGLU, 0, ybuf,
                               SPIRAL_TYPE_F32, wbuf, 4096, nullptr) != SPIRAL_OK, "glu odd rows");
  EXPECT(spiral_mul_mat_id_glu(q, wbuf, 144, 4, 8, 32, xbuf, 1, ids, 4, 2, 77, 0, ybuf, SPIRAL_TYPE_F32, wbuf, 4096,
                               nullptr) == SPIRAL_ERR_TYPE, "glu op");
  EXPECT(spiral_mul_mat_id_glu_fits(q, big - 1, big - 31) == 0 || spiral_mul_mat_id_glu_fits(q, big - 1, big - 31) == 1,
         "glu_fits at max");
  EXPECT(spiral_glu(SPIRAL_GLU_SWIGLU, 0, ybuf, big, big / 2 + 1, 2, ybuf, big, nullptr) != SPIRAL_OK,
         "glu overflow");
  EXPECT(spiral_glu(SPIRAL_GLU_SWIGLU, 2, ybuf, 8, 4, 2, ybuf, 4, nullptr) == SPIRAL_ERR_TYPE, "glu swapped");
  EXPECT(spiral_glu_split(SPIRAL_GLU_SWIGLU, 0, ybuf, big, ybuf, 8, 4, big, ybuf, 8, nullptr) != SPIRAL_OK,
         "glu_split overflow");
  EXPECT(spiral_glu_split(SPIRAL_GLU_SWIGLU, 0, ybuf, 2, ybuf, 8, 4, 2, ybuf, 8, nullptr) == SPIRAL_ERR_SHAPE,
         "glu_split ld");
  EXPECT(spiral_glu_split(SPIRAL_GLU_SWIGLU, 0, nullptr, 8, ybuf, 8, 4, 2, ybuf, 8, nullptr) == SPIRAL_ERR_NULL,
         "glu_split null");
  EXPECT(spiral_glu(SPIRAL_GLU_SWIGLU_OAI, 0, ybuf, 8, 4, 2, ybuf, 4, nullptr) == SPIRAL_ERR_TYPE, "glu oai plain");
  EXPECT(spiral_glu_swiglu_oai(0, 1.702f, 7.0f, ybuf, big, big / 2 + 1, 2, ybuf, big, nullptr) != SPIRAL_OK,
         "glu oai overflow");
  EXPECT(spiral_glu_split_swiglu_oai(0, 1.702f, 7.0f, ybuf, big, ybuf, 8, 4, big, ybuf, 8, nullptr) != SPIRAL_OK,
         "glu_split oai overflow");
  EXPECT(spiral_glu_split_swiglu_oai(1, 1.702f, 7.0f, ybuf, 8, nullptr, 8, 4, 2, ybuf, 8, nullptr) ==
             SPIRAL_ERR_NULL, "glu_split oai null");
  EXPECT(spiral_mul_mat_id_glu_split(q, wbuf, nullptr, 144, 4, 4, 32, xbuf, 1, ids, 4, 2, SPIRAL_GLU_SWIGLU, 0, ybuf,
                                     SPIRAL_TYPE_F32, wbuf, 4096, nullptr) == SPIRAL_ERR_NULL, "glu_split null up");
  EXPECT(spiral_mul_mat_id_glu_split(q, wbuf, wbuf, big, 4, big / 2 + 1, 32, xbuf, 1, ids, 4, 2, SPIRAL_GLU_SWIGLU, 0,
                                     ybuf, SPIRAL_TYPE_F32, wbuf, 4096, nullptr) != SPIRAL_OK, "glu_split at max");
  EXPECT(spiral_mul_mat_id_glu_split(q, wbuf, wbuf + 2, 144, 4, 4, 32, xbuf, 1, ids, 4, 2, SPIRAL_GLU_SWIGLU, 0, ybuf,
                                     SPIRAL_TYPE_F32, wbuf, 4096, nullptr) != SPIRAL_OK, "glu_split align");
  EXPECT(quants_unpack_all(q, nullptr, 64, 8, xbuf, nullptr) != SPIRAL_OK, "unpack_all null");
  EXPECT(quants_unpack_mmul_all(q, wbuf, xbuf, nullptr, 64, 8, nullptr) != SPIRAL_OK, "unpack_mmul_all null");

  // ggml surface with no buffer.
  spiral_tensor a{}, b{}, c{};
  a.type = q;
  a.ne[0] = 4096;
  a.ne[1] = 8;
  a.ne[2] = a.ne[3] = 1;
  a.nb[0] = 18;
  a.nb[1] = 4096 / 32 * 18;
  a.nb[2] = a.nb[3] = a.nb[1] * 8;
  b.type = SPIRAL_TYPE_F32;
  b.ne[0] = 4096;
  b.ne[1] = b.ne[2] = b.ne[3] = 1;
  b.nb[0] = 4;
  b.nb[1] = b.nb[2] = b.nb[3] = 4096 * 4;
  c = b;
  c.ne[0] = 8;
  c.op = SPIRAL_OP_MUL_MAT;
  c.src[0] = &a;
  c.src[1] = &b;
  EXPECT(spiral_supports_op(&c) == 0, "supports_op without a buffer");
  EXPECT(spiral_supports_op(nullptr) == 0, "supports_op null");
  for (int op = -3; op < 12; ++op) {
    c.op = op;
    (void)spiral_supports_op(&c);
  }
  for (int64_t ne0 : {int64_t(-32), int64_t(0), int64_t(31), big, big - 31}) {
    a.ne[0] = ne0;
    (void)spiral_buft_alloc_size(&a);
    c.op = SPIRAL_OP_MUL_MAT;
    (void)spiral_supports_op(&c);
  }
  a.ne[0] = 4096;
  a.ne[1] = big;
  (void)spiral_buft_alloc_size(&a);
  EXPECT(spiral_buft_alloc_size(nullptr) == 0, "alloc_size null");
  EXPECT(spiral_buffer_init_tensor(nullptr, &a) != SPIRAL_OK, "init_tensor null buffer");
  EXPECT(spiral_buffer_set_tensor(nullptr, &a, wbuf, 0, 16) != SPIRAL_OK, "set_tensor null buffer");
  EXPECT(spiral_buffer_get_tensor(nullptr, &a, wbuf, 0, 16) != SPIRAL_OK, "get_tensor null buffer");
  EXPECT(spiral_buffer_memset_tensor(nullptr, &a, 0, 0, 16) != SPIRAL_OK, "memset_tensor null buffer");
  EXPECT(spiral_buffer_clear(nullptr, 0) != SPIRAL_OK, "clear null buffer");
  EXPECT(spiral_buffer_get_base(nullptr) == nullptr && spiral_buffer_get_size(nullptr) == 0, "buffer getters");
  spiral_buffer_free(nullptr);
  spiral_tensor* nodes[1] = {&c};
  spiral_cgraph g{1, nodes};
  EXPECT(spiral_backend_graph_compute(nullptr, &g) != SPIRAL_OK, "graph_compute null backend");
  EXPECT(spiral_backend_synchronize(nullptr) != SPIRAL_OK, "synchronize null backend");
  EXPECT(spiral_backend_stream(nullptr) == nullptr, "stream null backend");
  spiral_backend_free(nullptr);
}


// ---- the llama.cpp shim's conversion ----------------
// A minimal ggml_tensor with the fields the shim reads (ggml.h's names).
struct ggml_tensor_mock {
  int type;
  void* buffer;  // ggml_backend_buffer_t; the shim maps ->context, NULL here
  int64_t ne[4];
  size_t nb[4];
  int op;
  int32_t op_params[16];
  int32_t flags;
  ggml_tensor_mock* src[10];
  ggml_tensor_mock* view_src;
  size_t view_offs;
  void* data;
  char name[64];
};

struct shim_node {
  spiral_tensor t, src[SPIRAL_MAX_SRC], owner, src_owner[SPIRAL_MAX_SRC];
};

void shim_copy_fields(const ggml_tensor_mock* t, spiral_tensor* s) {
  std::memset(s, 0, sizeof(*s));
  s->type = t->type;
  s->buffer = nullptr;
  for (int i = 0; i < 4; ++i) {
    s->ne[i] = t->ne[i];
    s->nb[i] = t->nb[i];
  }
  s->op = t->op;  // the mock carries spiral's op ids already
  std::memcpy(s->op_params, t->op_params, sizeof(s->op_params));
  s->flags = t->flags;
  s->data = t->data;
  s->view_offs = t->view_offs;
  std::strncpy(s->name, t->name, SPIRAL_MAX_NAME - 1);
}

void shim_to_spiral1(const ggml_tensor_mock* t, spiral_tensor* s, spiral_tensor* owner) {
  shim_copy_fields(t, s);
  if (t->view_src) {
    shim_copy_fields(t->view_src, owner);
    s->view_src = owner;
  }
}

void shim_to_spiral(const ggml_tensor_mock* t, shim_node* n) {
  shim_to_spiral1(t, &n->t, &n->owner);
  for (int i = 0; i < SPIRAL_MAX_SRC; ++i)
    if (t->src[i]) {
      shim_to_spiral1(t->src[i], &n->src[i], &n->src_owner[i]);
      n->t.src[i] = &n->src[i];
    }
}

ggml_tensor_mock mock_tensor(int type, int64_t ne0, int64_t ne1, int64_t ne2, size_t row_bytes, size_t elem,
                             void* data, const char* name) {
  ggml_tensor_mock t;
  std::memset(&t, 0, sizeof(t));
  t.type = type;
  t.ne[0] = ne0;
  t.ne[1] = ne1;
  t.ne[2] = ne2;
  t.ne[3] = 1;
  t.nb[0] = elem;
  t.nb[1] = row_bytes;
  t.nb[2] = row_bytes * static_cast<size_t>(ne1);
  t.nb[3] = t.nb[2] * static_cast<size_t>(ne2);
  t.data = data;
  std::strncpy(t.name, name, sizeof(t.name) - 1);
  return t;
}

void check_shim() {
  const int q = SPIRAL_TYPE_Q4_0;
  const int64_t k = 256, rows = 64, experts = 4;
  const size_t rb = static_cast<size_t>(spiral_row_bytes(q, k));
  std::vector<uint8_t> weight(rb * rows * experts), act(4096), out(4096), idsb(256);
  // The owner: an expert stack [experts][rows][k] of Q4_0.
  ggml_tensor_mock w = mock_tensor(q, k, rows, experts, rb, 18, weight.data(), "blk.0.ffn_gate_exps.weight");
  // A row view (rows 8..39 of expert 0) and a whole-expert view (expert 2).
  ggml_tensor_mock rowv = mock_tensor(q, k, 32, 1, rb, 18, weight.data() + 8 * rb, "rows");
  rowv.op = SPIRAL_OP_VIEW;
  rowv.view_src = &w;
  rowv.view_offs = 8 * rb;
  ggml_tensor_mock expv = mock_tensor(q, k, rows, 1, rb, 18, weight.data() + 2 * rows * rb, "expert 2");
  expv.op = SPIRAL_OP_VIEW;
  expv.view_src = &w;
  expv.view_offs = 2 * rows * rb;
  ggml_tensor_mock x = mock_tensor(SPIRAL_TYPE_F32, k, 1, 1, k * 4, 4, act.data(), "x");
  ggml_tensor_mock ids = mock_tensor(SPIRAL_TYPE_I32, 2, 1, 1, 8, 4, idsb.data(), "ids");

  for (const ggml_tensor_mock* a : {&w, &rowv, &expv}) {
    ggml_tensor_mock mm = mock_tensor(SPIRAL_TYPE_F32, a->ne[1], 1, 1, a->ne[1] * 4, 4, out.data(), "mul_mat");
    mm.op = SPIRAL_OP_MUL_MAT;
    mm.src[0] = const_cast<ggml_tensor_mock*>(a);
    mm.src[1] = &x;
    ggml_tensor_mock gr = mock_tensor(SPIRAL_TYPE_F32, k, 2, 1, k * 4, 4, out.data(), "get_rows");
    gr.op = SPIRAL_OP_GET_ROWS;
    gr.src[0] = const_cast<ggml_tensor_mock*>(a);
    gr.src[1] = &ids;
    for (ggml_tensor_mock* node : {&mm, &gr}) {
      // Storage as a caller's stack would leave it: garbage, then the shim.
      shim_node* n = static_cast<shim_node*>(std::malloc(sizeof(shim_node)));
      std::memset(n, 0xA5, sizeof(shim_node));
      shim_to_spiral(node, n);
      EXPECT(n->t.src[0] == &n->src[0] && n->t.src[1] == &n->src[1] && n->t.src[2] == nullptr, "shim srcs");
      EXPECT(n->t.view_src == nullptr, "shim node view_src");
      if (a->view_src) {
        EXPECT(n->src[0].view_src == &n->src_owner[0] && n->src[0].view_offs == a->view_offs, "shim view mapped");
        EXPECT(n->src_owner[0].data == weight.data() && n->src_owner[0].view_src == nullptr, "shim owner");
      } else {
        EXPECT(n->src[0].view_src == nullptr, "shim no view");
      }
      EXPECT(std::strcmp(n->src[0].name, a->name) == 0, "shim name");
      // No buffer: the op is not supported, but supports_op reads every
      // field (view_src included) without touching garbage.
      EXPECT(spiral_supports_op(&n->t) == 0, "shim supports_op without a buffer");
      EXPECT(spiral_buft_alloc_size(&n->src[0]) == static_cast<size_t>(a->ne[1] * a->ne[2]) * rb, "shim alloc_size");
      EXPECT(spiral_buffer_init_tensor(nullptr, &n->src[0]) == SPIRAL_ERR_NULL, "shim init_tensor null buffer");
      std::free(n);
    }
  }
}

}  // namespace

int main() {
  std::setvbuf(stdout, nullptr, _IOLBF, 0);
  check_repack();
  std::printf("repack checks done (%d failures so far)\n", g_failures);
  check_oracle();
  std::printf("oracle and CPU-baseline checks done (%d failures so far)\n", g_failures);
  check_shim();
  std::printf("shim checks done (%d failures so far)\n", g_failures);
  check_validation();
  std::printf("validation checks done: %d failures\n", g_failures);
  return g_failures == 0 ? 0 : 1;
}
