// Dequant-GEMM on bf16 MFMA: Y[m][n] = sum_k X[m][k] * W[n][k] for planar
// quantized W (any of Q4_0 / Q8_0 / Q6_K), bf16 X, fp32 accumulation.
//
// This is the prefill form of the reference's fused unpack + mmul
// (src/quants/q4_0/mmul.aie.h:16-90 with aie::mmul<4,8,8,bf16,bf16>,
// src/quants/common/mmul.aie.h:9-22): weights are dequantized exactly to bf16
// and multiplied against bf16 inputs with fp32 accumulation, so each product
// term equals the reference's; only the fp32 summation order differs.
//
// Two launches on the caller's stream:
//  1. pack_x_kernel rewrites X into MFMA A-operand order in the caller's
//     workspace: 1 KiB fragments Xp[m / 16][k / 32][lane][8], lane l holding
//     row l % 16, k 8 (l / 16) .. + 7 of its 16 x 32 block. A wave then loads
//     one fragment as 1 KiB of consecutive bytes (eight whole 128-byte lines),
//     where loading it from X directly touches 16 rows x 64 bytes; on gfx950
//     the latter pattern reaches about a third of the L2 -> CU throughput.
//  2. gemm_kernel: one workgroup per 128 (m) x 64 (n) tile of Y (m = 512,
//     n = 4096: 256 tiles, one per CU), 8 waves, k steps of 128.
//      - The step's 64 x 128 weight tile is dequantized once per workgroup
//        into LDS (each of the 512 threads turns one 16-element piece); LDS
//        holds four such tiles, the one being read and the next three.
//      - Wave (mw, q) = (w % 2, w / 2) owns rows 64 mw .. + 63 of the tile
//        and the k-quarter q (32 wide, one MFMA depth) of every step: four
//        X fragments (buffer loads from the packed workspace, no LDS) and
//        four B fragments from LDS feed 16 v_mfma_f32_16x16x32_bf16. Each
//        weight element is read from LDS by two waves, each X element by one.
//      - Register rings keep X three steps and weights five steps ahead
//        (Q6_K: one and three).
//        Step s + 2's weights are dequantized while step s multiplies, so a
//        barrier is needed only after every second step.
//      - Scheduling fences keep each step's MFMAs, LDS reads, dequantization
//        and loads together; without them the compiler hoists later steps'
//        dequantization above the loads it waits for.
//      - The four k-quarters are summed through LDS at the end; each wave
//        then stages its 16 x 64 output block in LDS and writes it as 16-byte
//        row pieces (1.7 us faster than per-element stores at M = 512).
//  Workgroups are numbered so that each XCD (dispatch is round-robin over the
//  8 XCDs) gets a contiguous range of tiles sharing X rows in its L2.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "dequant_impl.h"

namespace spiral {
int64_t gemm_max_k();

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int kBM = 128, kBN = 64, kBK = 128, kThreads = 512;
constexpr int kPitch = kBK + 8;  // LDS row pitch in bf16; the pad spreads rows over banks
constexpr int kRing = 4;
constexpr int kBTile = kBN * kPitch;                   // one weight tile in LDS (bf16)
constexpr int kRedFloats = 2 * 4 * 3 * 16 * 64;        // k-quarter partials (floats)
constexpr int64_t kMaxBufferBytes = int64_t(1) << 31;  // buffer offsets are 32-bit
static_assert(4 * kBTile * 2 <= kRedFloats * 4, "weight tiles and partials share one LDS array");

// Tile index for workgroup b of `grid`: consecutive workgroups go to
// consecutive XCDs, so hand XCD x the tiles [x grid / 8, (x + 1) grid / 8).
__device__ __forceinline__ int64_t xcd_tile(int64_t b, int64_t grid) {
  if (grid % 8 != 0) return b;
  return (b % 8) * (grid / 8) + b / 8;
}

// Xp[mb][kk][lane][8] = X[16 mb + lane % 16][32 kk + 8 (lane / 16) + e];
// rows past m are zero. Wave w of the grid writes fragment f = w (1 KiB of
// consecutive bytes, one store); its lanes read their 16 bytes straight from
// X. The pass moves 2 x 4 MiB at m = 512, k = 4096, so the latency of one
// load and one store per lane is what it costs: no LDS tile, no barrier.
__global__ void __launch_bounds__(256) pack_x_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t m,
                                                     int64_t k, uint16_t* __restrict__ xp) {
  const uint32_t kk_n = static_cast<uint32_t>(k >> 5);
  const uint32_t frags = static_cast<uint32_t>((m + 15) >> 4) * kk_n;
  const uint32_t f = blockIdx.x * 4u + (threadIdx.x >> 6), lane = threadIdx.x & 63u;
  if (f >= frags) return;
  const uint32_t mb = f / kk_n, kk = f - mb * kk_n;
  const int64_t r = 16 * static_cast<int64_t>(mb) + (lane & 15u);
  uint4 v = make_uint4(0u, 0u, 0u, 0u);
  if (r < m) v = *reinterpret_cast<const uint4*>(x + r * ldx + 32 * kk + 8 * (lane >> 4));
  *reinterpret_cast<uint4*>(xp + (static_cast<int64_t>(f) * 64 + lane) * 8) = v;
}

// The four X fragments (m-blocks) of a wave for one k-quarter.
struct AFrag {
  uint4 v[4];
};

// voff[i]: the lane's byte offset of m-block i's fragment row in the packed
// workspace (blocks past m clamped: their outputs are never stored); the
// k32 index k0 / 32 becomes the scalar offset.
__device__ __forceinline__ void load_a(AFrag& a, __amdgpu_buffer_rsrc_t X, const uint32_t (&voff)[4], int64_t k0,
                                       bool valid = true) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
    a.v[i] = valid ? bload16(X, voff[i], static_cast<uint32_t>(k0 >> 5) * 1024u) : make_uint4(0u, 0u, 0u, 0u);
}

template <int TYPE>
__device__ __forceinline__ void store_b(const Piece<TYPE>& pc, const typename Piece<TYPE>::Addr& pa, uint16_t* bs,
                                        int tid) {
  uint4 o0, o1;
  pc.dequant(pa, o0, o1);
  uint16_t* dst = bs + (tid >> 3) * kPitch + 16 * (tid & 7);
  *reinterpret_cast<uint4*>(dst) = o0;
  *reinterpret_cast<uint4*>(dst + 8) = o1;
}

// B operands of k-quarter q for the 64 columns: lane l takes column
// 16 j + l % 16, k = 32 q + 8 (l / 16) .. + 7.
struct BFrag {
  bf16x8_t b[4];
};

__device__ __forceinline__ void read_bfrag(BFrag& f, const uint16_t* bs, int q, int lane) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
    f.b[j] = *reinterpret_cast<const bf16x8_t*>(bs + (16 * j + (lane & 15)) * kPitch + 32 * q + 8 * (lane >> 4));
}

__device__ __forceinline__ void mfma_step(f32x4_t (&acc)[4][4], const AFrag& a, const BFrag& b) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bf16x8_t av = __builtin_bit_cast(bf16x8_t, a.v[i]);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b.b[j], acc[i][j], 0, 0, 0);
  }
}

// Register rings: kARing<TYPE> X slots loaded kARing - 1 steps ahead and
// kWRing<TYPE> weight-piece slots loaded kWRing + 1 steps ahead. Q6_K
// pieces take twice the registers of the others, so its rings are shorter.
template <int TYPE>
constexpr int kARing = (TYPE == SPIRAL_TYPE_Q6_K || is_kquant(TYPE) || TYPE == SPIRAL_TYPE_IQ4_XS) ? 2 : 4;
template <int TYPE>
constexpr int kWRing = (TYPE == SPIRAL_TYPE_Q6_K || is_kquant(TYPE) || TYPE == SPIRAL_TYPE_IQ4_XS) ? 2 : 4;

template <int TYPE>
struct Pipe {
  AFrag a[kARing<TYPE>];
  Piece<TYPE> pc[kWRing<TYPE>];
};

// Step s (d = s % 4: LDS tile of step s): request X of step s + A - 1 (A =
// kARing, slot (s - 1) % A, free since step s - 1) and weights of step
// s + R + 1 (R = kWRing, slot (s + 1) % R, free since step s - 1), both
// clamped to the last full step; read step s's B operands, multiply X slot
// s % A, dequantize step s + 2 (slot (s + 2) % R) into tile (s + 2) % 4.
// Tile (s + 2) % 4 was last read at step s - 2 and tile s % 4 was written at
// step s - 2, so one barrier after every odd step orders both.
template <int TYPE>
__device__ __forceinline__ void gemm_step(f32x4_t (&acc)[4][4], Pipe<TYPE>& pp, uint16_t* bs0, int d, int s,
                                          int full, __amdgpu_buffer_rsrc_t X, const uint32_t (&voff)[4],
                                          const Planes& P, const typename Piece<TYPE>::Addr& pa, int q, int tid,
                                          int lane) {
  constexpr int A = kARing<TYPE>, R = kWRing<TYPE>;
  load_a(pp.a[(d + A - 1) % A], X, voff, static_cast<int64_t>(min(s + A - 1, full - 1)) * kBK + 32 * q);
  pp.pc[(d + 1) % R].load(P, pa, static_cast<int64_t>(min(s + R + 1, full - 1)) * kBK);
  BFrag b;
  read_bfrag(b, bs0 + d * kBTile, q, lane);
  mfma_step(acc, pp.a[d % A], b);
  store_b<TYPE>(pp.pc[(d + 2) % R], pa, bs0 + ((d + 2) % kRing) * kBTile, tid);
  __builtin_amdgcn_sched_barrier(0);
  if (d & 1) __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
}

template <int TYPE, bool F32_OUT>
__global__ void __launch_bounds__(kThreads) gemm_kernel(const uint8_t* __restrict__ w, int64_t n_rows, int64_t k,
                                                        const uint16_t* __restrict__ xp, int64_t m,
                                                        void* __restrict__ y, int64_t ldy, int64_t n_tiles_n) {
  // Four weight tiles during the loop; the k-quarter partial sums after it.
  __shared__ __align__(16) float smem[kRedFloats];
  uint16_t* Bs = reinterpret_cast<uint16_t*>(smem);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int mw = wave & 1, q = wave >> 1;
  const int64_t tile = xcd_tile(blockIdx.x, gridDim.x);
  const int64_t m0 = (tile / n_tiles_n) * kBM, n0 = (tile % n_tiles_n) * kBN;
  const int64_t row0 = m0 + 64 * mw;
  const int64_t nb = k / block_elems(TYPE);
  // 32-bit step counters keep the ring's clamps scalar (k is at most
  // gemm_max_k(), so k / 128 fits)
  const int full = static_cast<int>(k / kBK);
  const int tail = static_cast<int>(k - full * kBK);  // 0, 32, 64 or 96

  const int64_t kk_n = k >> 5, mb_n = (m + 15) >> 4;
  const __amdgpu_buffer_rsrc_t X = buffer_rsrc(xp, static_cast<uint32_t>(mb_n * kk_n * 1024));
  uint32_t voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    voff[i] = static_cast<uint32_t>(min((row0 >> 4) + i, mb_n - 1) * kk_n * 1024 + lane * 16);
  const Planes P = make_planes<TYPE>(w, n_rows, nb);
  const typename Piece<TYPE>::Addr pa = Piece<TYPE>::addr(min(n0 + (tid >> 3), n_rows - 1), nb, tid & 7);

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  if (full > 0) {
    constexpr int A = kARing<TYPE>, R = kWRing<TYPE>;
    Pipe<TYPE> pp;
#pragma unroll
    for (int i = 0; i < A - 1; ++i) load_a(pp.a[i], X, voff, static_cast<int64_t>(min(i, full - 1)) * kBK + 32 * q);
#pragma unroll
    for (int i = 0; i < R; ++i) pp.pc[i].load(P, pa, static_cast<int64_t>(min(i, full - 1)) * kBK);
    store_b<TYPE>(pp.pc[0], pa, Bs, tid);
    store_b<TYPE>(pp.pc[1], pa, Bs + kBTile, tid);
    pp.pc[0].load(P, pa, static_cast<int64_t>(min(R, full - 1)) * kBK);
    __syncthreads();
    int s0 = 0;
    for (; s0 + kRing <= full; s0 += kRing) {
#pragma unroll
      for (int d = 0; d < kRing; ++d) gemm_step<TYPE>(acc, pp, Bs, d, s0 + d, full, X, voff, P, pa, q, tid, lane);
    }
#pragma unroll
    for (int d = 0; d < kRing - 1; ++d) {
      if (s0 + d < full) gemm_step<TYPE>(acc, pp, Bs, d, s0 + d, full, X, voff, P, pa, q, tid, lane);
    }
    __syncthreads();
  }
  if (tail > 0) {
    // k tail of 32, 64 or 96: pieces past it and k-quarters past it are zero.
    Piece<TYPE> pt;
    AFrag at;
    if (16 * (tid & 7) < tail)
      pt.load(P, pa, full * kBK);
    else
      pt.zero();
    load_a(at, X, voff, full * kBK + 32 * q, 32 * q < tail);
    store_b<TYPE>(pt, pa, Bs, tid);
    __syncthreads();
    BFrag bt;
    read_bfrag(bt, Bs, q, lane);
    mfma_step(acc, at, bt);
    __syncthreads();
  }

  // Sum the k-quarters: wave (mw, q) owns output m-block q of its 64 rows.
  // It parks its other three m-blocks in LDS (slot: the writer's rank among
  // the three non-owners), then adds the three partials of its own block.
  float* red = smem;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (i == q) continue;
    float* dst = red + ((mw * 4 + i) * 3 + (q < i ? q : q - 1)) * (16 * 64);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[(j * 4 + e) * 64 + lane] = acc[i][j][e];
  }
  __syncthreads();
  f32x4_t out[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (i != q) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = acc[i][j];
  }
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    const float* src = red + ((mw * 4 + q) * 3 + t) * (16 * 64);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) out[j][e] += src[(j * 4 + e) * 64 + lane];
  }

  // The wave's 16 x 64 output block goes through LDS (accumulator layout:
  // lane l holds D[4 (l / 16) + e][16 j + l % 16]) so that it leaves as
  // 16-byte row pieces instead of 2- or 4-byte scattered stores. Each wave
  // uses its own region, after every wave has read the partials above.
  using OutT = typename std::conditional<F32_OUT, float, __bf16>::type;
  constexpr int kPer = 16 / sizeof(OutT);           // elements per 16-byte piece
  constexpr int kTPitch = 64 + kPer;                // padded row, in elements
  __syncthreads();
  OutT* T = reinterpret_cast<OutT*>(smem) + wave * 16 * kTPitch;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) T[(4 * (lane >> 4) + e) * kTPitch + 16 * j + (lane & 15)] = static_cast<OutT>(out[j][e]);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  constexpr int kPieces = 16 * 64 / kPer;           // per wave: 128 (bf16) or 256 (f32)
#pragma unroll
  for (int h = 0; h < kPieces / 64; ++h) {
    const int c = lane + 64 * h;
    const int r = c / (64 / kPer), col = (c % (64 / kPer)) * kPer;
    const int64_t gm = row0 + 16 * q + r, gn = n0 + col;
    if (gm >= m) continue;
    const uint4 v = *reinterpret_cast<const uint4*>(T + r * kTPitch + col);
    OutT* dst = static_cast<OutT*>(y) + gm * ldy + gn;
    if (gn + kPer <= n_rows && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
      *reinterpret_cast<uint4*>(dst) = v;
    } else {
      const OutT* src = T + r * kTPitch + col;
      for (int i = 0; i < kPer && gn + i < n_rows; ++i) dst[i] = src[i];
    }
  }
}

// Rows of X per launch: the packed chunk (rows rounded up to 16, times k
// bf16) stays below 2 GiB so buffer offsets fit in 32 bits.
// k is at most gemm_max_k(), so one M tile of packed X fits.
int64_t chunk_rows(int64_t k) { return std::max<int64_t>(kBM, (kMaxBufferBytes / (k * 2)) / kBM * kBM); }

template <int TYPE>
int launch_gemm(const void* w, int64_t n_rows, int64_t k, const uint16_t* x, int64_t ldx, int64_t m, void* y,
                int y_type, int64_t ldy, uint16_t* xp, hipStream_t s) {
  // Weight planes are addressed with 32-bit offsets (the largest plane is at
  // most 16/18 of the tensor).
  const int64_t wbytes = spiral_tensor_bytes(TYPE, n_rows, k);
  if (wbytes == 0 || wbytes >= kMaxBufferBytes * 2 || k > gemm_max_k()) return SPIRAL_ERR_SHAPE;
  const int64_t chunk = chunk_rows(k);
  const int64_t tn = ceil_div(n_rows, kBN);
  const uint8_t* W = static_cast<const uint8_t*>(w);
  const int64_t ysz = y_type == SPIRAL_TYPE_F32 ? 4 : 2;
  for (int64_t mo = 0; mo < m; mo += chunk) {
    const int64_t mc = std::min(chunk, m - mo);
    const int64_t tm = ceil_div(mc, kBM);
    const int64_t packs = ceil_div(ceil_div(mc, 16) * (k >> 5), 4);
    if (tn * tm > INT32_MAX || packs > INT32_MAX) return SPIRAL_ERR_SHAPE;
    hipLaunchKernelGGL(pack_x_kernel, dim3(static_cast<unsigned>(packs)), dim3(256), 0, s, x + mo * ldx, ldx, mc, k,
                       xp);
    int rc = launch_status();
    if (rc != SPIRAL_OK) return rc;
    const dim3 grid(static_cast<unsigned>(tn * tm));
    void* yc = static_cast<uint8_t*>(y) + mo * ldy * ysz;
    if (y_type == SPIRAL_TYPE_F32)
      hipLaunchKernelGGL((gemm_kernel<TYPE, true>), grid, dim3(kThreads), 0, s, W, n_rows, k, xp, mc, yc, ldy, tn);
    else
      hipLaunchKernelGGL((gemm_kernel<TYPE, false>), grid, dim3(kThreads), 0, s, W, n_rows, k, xp, mc, yc, ldy, tn);
    rc = launch_status();
    if (rc != SPIRAL_OK) return rc;
  }
  return SPIRAL_OK;
}

}  // namespace

// Longest row the GEMM takes: one 128-row tile of packed X must fit a
// 32-bit buffer offset.
int64_t gemm_max_k() { return kMaxBufferBytes / (2 * kBM); }

// Workspace for the packed X of one launch chunk (0 when k > gemm_max_k()).
int64_t gemm_workspace_bytes(int64_t m, int64_t k) {
  if (k <= 0 || k > gemm_max_k()) return 0;
  const int64_t rows = std::min(m, chunk_rows(k));
  return ceil_div(rows, 16) * 16 * k * 2;
}

// Y = X W^T; arguments validated by the caller (k a multiple of the block, x
// rows 16-byte aligned with ldx a multiple of 8, workspace of at least
// gemm_workspace_bytes(m, k) bytes, 16-byte aligned).
int gemm(int type, const void* w, int64_t n_rows, int64_t k, const uint16_t* x, int64_t ldx, int64_t m, void* y,
         int y_type, int64_t ldy, void* workspace, hipStream_t s) {
  uint16_t* xp = static_cast<uint16_t*>(workspace);
  switch (type) {
    case SPIRAL_TYPE_Q4_0: return launch_gemm<SPIRAL_TYPE_Q4_0>(w, n_rows, k, x, ldx, m, y, y_type, ldy, xp, s);
    case SPIRAL_TYPE_Q8_0: return launch_gemm<SPIRAL_TYPE_Q8_0>(w, n_rows, k, x, ldx, m, y, y_type, ldy, xp, s);
    case SPIRAL_TYPE_Q6_K: return launch_gemm<SPIRAL_TYPE_Q6_K>(w, n_rows, k, x, ldx, m, y, y_type, ldy, xp, s);
    case SPIRAL_TYPE_Q4_K: return launch_gemm<SPIRAL_TYPE_Q4_K>(w, n_rows, k, x, ldx, m, y, y_type, ldy, xp, s);
    case SPIRAL_TYPE_Q5_K: return launch_gemm<SPIRAL_TYPE_Q5_K>(w, n_rows, k, x, ldx, m, y, y_type, ldy, xp, s);
    case SPIRAL_TYPE_IQ4_NL: return launch_gemm<SPIRAL_TYPE_IQ4_NL>(w, n_rows, k, x, ldx, m, y, y_type, ldy, xp, s);
    case SPIRAL_TYPE_IQ4_XS: return launch_gemm<SPIRAL_TYPE_IQ4_XS>(w, n_rows, k, x, ldx, m, y, y_type, ldy, xp, s);
    default: return SPIRAL_ERR_TYPE;
  }
}

}  // namespace spiral
