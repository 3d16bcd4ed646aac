// Grouped dequant-GEMM for MUL_MAT_ID at prefill sizes (many routed tokens
// per expert), ggml's mul_mat_id over expert-stacked quantized weights.
//
// Three launches on the caller's stream, after route_kernel has sorted the
// (token, slot) pairs by expert (offsets / list) and counted each expert's
// 16-row blocks (blk_base) and 128-row m-tiles (mt_base):
//  1. moe_pack_kernel gathers each expert's routed activation rows into MFMA
//     A-operand order in the workspace: 1 KiB fragments Xp[block][k / 32]
//     [lane][8], lane l holding routed row l % 16 of the block. Fragment
//     (block, 4 st + s) holds, for lane group g, the elements
//     MoePiece<TYPE>::local(g, s, 0..7) of k step st: the order in which the
//     streaming MUL_MAT_ID kernel stages them. Rows past an expert's count
//     are zero.
//  2. moe_gemm_kernel: workgroup (m-tile, n-part): the m-tile is up to 128 of
//     one expert's routed rows (8 MFMA row blocks), the n-part a contiguous
//     range of 64-column n-tiles of that expert's matrix. The workgroup
//     streams (n-tile, k step) units end to end, so its loads run ahead
//     across n-tile ends:
//      - each unit's 64 x 128 weight tile is dequantized once into LDS (four
//        stages: the one being read and the next three), each thread turning
//        half a MoePiece (two of its four MFMA groups of eight);
//      - wave (h, q) = (w / 4, w % 4) owns half h of the m-tile's row blocks
//        (split evenly, so both waves of a SIMD multiply) and MFMA group q of
//        every step (the k-quarter that MoePiece::dequant(q) feeds): up to
//        four packed X fragments (buffer loads, no LDS) and four B operands
//        from LDS feed up to 16 v_mfma_f32_16x16x32_bf16; row blocks past the
//        m-tile's rows issue no loads and no MFMAs;
//      - at an n-tile's end the four k-quarter partials of each output block
//        meet in LDS and are summed as (q0 + q1) + (q2 + q3), and each output
//        row leaves as 16-byte pieces to its (token, slot) row.
//     So each (pair, column) sum is formed from the same operands, in the
//     same order, as in the streaming kernel that takes decode-sized
//     batches: a prefill call equals the same tokens sent in small calls,
//     bit for bit.
// An expert's weights are dequantized once per m-tile (once for up to 128
// routed tokens) and each weight feeds up to 8 MFMA row blocks, where the
// streaming form's passes of 16..64 tokens re-read and re-dequantize them.
#include <algorithm>

#include "common.h"
#include "dequant_impl.h"
#include "moe_piece.h"

namespace spiral {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int kGThreads = 512;
constexpr int kGMTile = 128;                 // routed rows per m-tile (8 row blocks)
constexpr int kGBN = 64;                     // weight rows (output columns) per n-tile
constexpr int kGPitch = 128 + 8;             // bf16 per LDS row of a dequantized step
constexpr int kGStage = kGBN * kGPitch;      // bf16 per LDS stage
constexpr int kGStages = 4;
constexpr int kGRed = 4 * 3 * 4 * 256;       // floats: k-quarter partials of one row-block half
constexpr int kGOutPitch = 64 + 4;           // floats per staged output row
constexpr int kGPackThreads = 256;
constexpr uint32_t kGSkip = 0x80000000u;     // buffer offset past every range: the load returns zero

// Grid: gridDim.y = experts, gridDim.x workgroups share an expert's
// fragments. Wave f of the expert packs fragment f, f + 4 gridDim.x, ...
template <int TYPE>
__global__ void __launch_bounds__(kGPackThreads) moe_pack_kernel(const uint16_t* __restrict__ x, int64_t k,
                                                                 int64_t x_slots, int64_t top_k,
                                                                 const int32_t* __restrict__ offsets,
                                                                 const int32_t* __restrict__ list,
                                                                 const int32_t* __restrict__ blk_base,
                                                                 uint16_t* __restrict__ xp) {
  const int32_t e = static_cast<int32_t>(blockIdx.y);
  const int32_t p0 = offsets[e], n_e = offsets[e + 1] - p0;
  if (n_e <= 0) return;
  const int64_t kk_n = k >> 5;
  const int64_t frags = static_cast<int64_t>((n_e + 15) >> 4) * kk_n;
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int64_t b0 = blk_base[e];
  for (int64_t f = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); f < frags;
       f += static_cast<int64_t>(gridDim.x) * 4) {
    const int64_t bl = f / kk_n, kk = f - bl * kk_n;
    const int st = static_cast<int>(kk >> 2), s = static_cast<int>(kk & 3);
    const int64_t i = bl * 16 + r;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (i < n_e) {
      const int64_t pr = list[p0 + i];
      const int64_t t = pr / top_k, slot = pr - t * top_k;
      const uint16_t* src = x + (t * x_slots + slot % x_slots) * k + 128 * static_cast<int64_t>(st);
      const int a = MoePiece<TYPE>::local(g, s, 0), b = MoePiece<TYPE>::local(g, s, 4);
      if (b == a + 4) {
        v = *reinterpret_cast<const uint4*>(src + a);
      } else {
        uint2 lo = *reinterpret_cast<const uint2*>(src + a), hi = *reinterpret_cast<const uint2*>(src + b);
        if constexpr (kStageSwap<TYPE>) {
          lo = stage_swap(lo);
          hi = stage_swap(hi);
        }
        v = make_uint4(lo.x, lo.y, hi.x, hi.y);
      }
    }
    *reinterpret_cast<uint4*>(xp + ((b0 + bl) * kk_n + kk) * 512 + lane * 8) = v;
  }
}

struct GFrag {
  uint4 v[4];
};

// Byte offsets in a format's first plane (the codes): of row `row`, and of
// k step st within a row.
template <int TYPE>
__device__ __forceinline__ uint32_t plane_a_row(int64_t nb) {
  if constexpr (TYPE == SPIRAL_TYPE_Q4_0 || TYPE == SPIRAL_TYPE_IQ4_NL) return static_cast<uint32_t>(nb * 16);
  else if constexpr (TYPE == SPIRAL_TYPE_Q8_0) return static_cast<uint32_t>(nb * 32);
  else return static_cast<uint32_t>(nb * 128);  // Q6_K ql, K-quant and IQ4_XS qs: 128 bytes a super-block
}
template <int TYPE>
__device__ __forceinline__ uint32_t plane_a_step(uint32_t st) {
  if constexpr (TYPE == SPIRAL_TYPE_Q4_0 || TYPE == SPIRAL_TYPE_IQ4_NL) return st * 64u;
  else if constexpr (TYPE == SPIRAL_TYPE_Q8_0) return st * 128u;
  else return (st >> 1) * 128u + (st & 1u) * 64u;
}

// Units ahead of the weight loads that a wave touches the weights' lines
// into L2: the register ring keeps only two pairs of units in flight, too
// few bytes to cover HBM latency on its own.
constexpr int kGPrefetch = 14;

// Unit cursor: (n-tile relative to the workgroup's first, k step).
struct GCur {
  int nt, st;
};

__device__ __forceinline__ void gadvance(GCur& c, int steps) {
  if (++c.st == steps) {
    c.st = 0;
    ++c.nt;
  }
}

template <int TYPE, bool F32_OUT>
__global__ void __launch_bounds__(kGThreads) moe_gemm_kernel(
    const uint8_t* __restrict__ w, int64_t expert_stride, int64_t n_rows, int64_t k, const uint16_t* __restrict__ xp,
    uint32_t xp_bytes, const int32_t* __restrict__ offsets, const int32_t* __restrict__ list,
    const int32_t* __restrict__ blk_base, const int32_t* __restrict__ mt_base, int32_t n_expert, int32_t parts,
    void* __restrict__ y) {
  __shared__ __align__(16) uint16_t Ws[kGStages * kGStage];
  __shared__ __align__(16) float red[kGRed];
  __shared__ __align__(16) float outs[8 * 16 * kGOutPitch];
  __shared__ int32_t s_pair[kGMTile];
  __shared__ int32_t s_e;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int mh = wave >> 2, q = wave & 3;

  // The `parts` workgroups of one m-tile are b, b + 8, ...: one XCD (dispatch
  // is round-robin over the 8 XCDs), so they share the m-tile's packed rows
  // in its L2.
  const int32_t b = static_cast<int32_t>(blockIdx.x);
  const int32_t mtile = (b / (8 * parts)) * 8 + b % 8, part = (b / 8) % parts;
  if (mtile >= mt_base[n_expert]) return;
  if (tid == 0) s_e = 0;
  __syncthreads();
  for (int32_t e = tid; e < n_expert; e += kGThreads)
    if (mt_base[e] <= mtile && mtile < mt_base[e + 1]) s_e = e;
  __syncthreads();
  const int32_t e = s_e;
  const int32_t p0 = offsets[e], rows0 = (mtile - mt_base[e]) * kGMTile;
  const int32_t nrow = min(kGMTile, offsets[e + 1] - p0 - rows0);  // at least 1
  const int mbv = (nrow + 15) >> 4;                                   // row blocks with routed rows
  // The row blocks are split evenly between the two halves of the waves, so
  // both waves of a SIMD multiply (a SIMD with one wave of MFMAs beside one
  // of dequantization alone runs far slower than either): half h takes
  // blocks hb[h] .. hb[h] + hn[h] - 1.
  const int hb1 = (mbv + 1) >> 1, hn0 = hb1, hn1 = mbv >> 1;
  const int mb0 = mh ? hb1 : 0, mbn = mh ? hn1 : hn0;  // this wave's blocks
  if (tid < kGMTile) s_pair[tid] = tid < nrow ? list[p0 + rows0 + tid] : -1;
  const int64_t n_tiles = (n_rows + kGBN - 1) / kGBN;
  const int64_t per = (n_tiles + parts - 1) / parts;
  const int64_t nt0 = part * per;
  const int n_nt = static_cast<int>(min(n_tiles, nt0 + per) - nt0);
  if (n_nt <= 0) return;

  const int64_t nb = k / block_elems(TYPE);
  const int S = static_cast<int>(k >> 7);  // 128-wide steps per n-tile
  const int U = n_nt * S;                  // units of this workgroup
  const uint32_t kk_n = static_cast<uint32_t>(k >> 5);
  const __amdgpu_buffer_rsrc_t X = buffer_rsrc(xp, xp_bytes);
  const int32_t pb = blk_base[e] + (rows0 >> 4);
  uint32_t voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    voff[i] = i < mbn ? static_cast<uint32_t>(pb + mb0 + i) * kk_n * 1024u + static_cast<uint32_t>(lane) * 16u
                      : kGSkip;
  }
  const Planes P = make_planes<TYPE>(w + e * expert_stride, n_rows, nb);
  // Weights go to LDS a pair of units at a time: this thread dequantizes the
  // piece of lane group gg, column cc of the pair's unit hh (waves 0..3 the
  // first unit, 4..7 the second); four consecutive lanes take the four
  // groups of one column (64 bytes of codes).
  const int hh = mh, gg = lane & 3, cc = 16 * (wave & 3) + (lane >> 2);

  const auto load_x = [&](GFrag& a, const GCur& c) __attribute__((always_inline)) {
    // past the last unit: reload the last one (never read); the step is
    // workgroup-uniform (a scalar offset)
    const uint32_t st = __builtin_amdgcn_readfirstlane(c.nt < n_nt ? c.st : S - 1);
    const uint32_t so = (4u * st + static_cast<uint32_t>(q)) * 1024u;
#pragma unroll
    for (int i = 0; i < 4; ++i) a.v[i] = bload16(X, voff[i], so);
  };
  const auto load_w = [&](MoePiece<TYPE>& pc, const GCur& c) __attribute__((always_inline)) {
    const bool in = c.nt < n_nt;
    const int64_t row = min((nt0 + (in ? c.nt : n_nt - 1)) * kGBN + cc, n_rows - 1);
    PieceAddr<TYPE> pa;
    pa.set(row, nb, gg);
    pa.load(pc, P, __builtin_amdgcn_readfirstlane(in ? c.st : S - 1));
  };
  // MFMA group s of the piece goes to k offset 32 s + 8 gg of the stage's
  // row cc: where lane group gg of the B operand of group s reads it.
  const auto dequant = [&](MoePiece<TYPE>& pc, int stage) __attribute__((always_inline)) {
    if constexpr (TYPE == SPIRAL_TYPE_Q4_0) {
      // the scale without a branch (the same value as prep()'s), so the
      // compiler can spread this among the MFMAs
      pc.m = fp16_scale(pc.d);
      pc.off = -1032.0f * pc.m;
      pc.off_hi = -72.0f * pc.m;
    } else {
      pc.prep();
    }
    uint16_t* dst = Ws + stage * kGStage + cc * kGPitch + 8 * gg;
#pragma unroll
    for (int s = 0; s < 4; ++s) *reinterpret_cast<uint4*>(dst + 32 * s) = pc.dequant(s);
  };
  const auto adv2 = [&](GCur& c) __attribute__((always_inline)) {
    gadvance(c, S);
    gadvance(c, S);
  };

  // L2 prefetch: at unit u, wave w touches the code lines of rows 8 w ..
  // 8 w + 7 of unit u + kGPrefetch (lane l takes row 8 w + l % 8; a dword
  // load brings in the line). The values are never used: each slot's result
  // is folded into `sink` four units later (by then it has arrived) and
  // sink is kept alive to the end, so the loads stay.
  const uint32_t pf_row = plane_a_row<TYPE>(nb);
  const uint32_t pf_voff = static_cast<uint32_t>(8 * wave + (lane & 7)) * pf_row;
  uint32_t pf[4] = {0u, 0u, 0u, 0u}, sink = 0u;
  GCur cp{0, 0};
#pragma unroll
  for (int i = 0; i < kGPrefetch; ++i) gadvance(cp, S);
  const auto prefetch = [&](int d) __attribute__((always_inline)) {
    sink |= pf[d];
    const uint32_t so = __builtin_amdgcn_readfirstlane(
        static_cast<uint32_t>(nt0 + cp.nt) * (kGBN * pf_row) + plane_a_step<TYPE>(static_cast<uint32_t>(cp.st)));
    pf[d] = bload4(P.a, pf_voff, so);
    gadvance(cp, S);
  };

  GFrag xa[4];
  MoePiece<TYPE> wr[2];  // pieces of the next two pairs
  GCur cx{0, 0}, cw{0, hh}, cc_{0, 0};  // X loads, weight loads (this thread's units), compute
  if (hh >= S) cw = GCur{1, hh - S};    // one-step n-tiles: unit 1 starts the next n-tile
  // Prologue: X of units 0..2; pieces of pairs 0 and 1, pair 0 dequantized
  // into stages 0 and 1, then the pieces of pair 2 in its slot.
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    load_x(xa[i], cx);
    gadvance(cx, S);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    load_w(wr[i], cw);
    adv2(cw);
  }
  dequant(wr[0], hh);
  load_w(wr[0], cw);
  adv2(cw);
  __syncthreads();

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // End of an n-tile: sum the k-quarters of each output block and store it.
  // Half hf's waves exchange through `red`: wave q owns the half's row
  // block q, the others park their partials of it (slot: the writer's rank
  // among the three non-owners).
  const auto epilogue = [&](int nt_rel) __attribute__((always_inline)) {
    using OutT = typename std::conditional<F32_OUT, float, __bf16>::type;
    constexpr int kPer = 16 / sizeof(OutT);  // elements per 16-byte piece
    const int64_t n0 = (nt0 + nt_rel) * kGBN;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int hfb = hf ? hb1 : 0, hfn = hf ? hn1 : hn0;  // half hf's blocks
      if (hfn == 0) break;
      if (mh == hf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (i == q || i >= hfn) continue;
          float* dst = red + (i * 3 + (q < i ? q : q - 1)) * (4 * 256);
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v) dst[(j * 4 + v) * 64 + lane] = acc[i][j][v];
        }
      }
      __syncthreads();
      if (mh == hf && q < hfn) {
        f32x4_t part4[4][4];  // [k-quarter][n-block]: the wave's own, the others' from red
#pragma unroll
        for (int o = 0; o < 4; ++o) {
          if (o == q) {
#pragma unroll
            for (int j = 0; j < 4; ++j) part4[o][j] = acc[o][j];
          } else {
            const float* src = red + (q * 3 + (o < q ? o : o - 1)) * (4 * 256);
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
              for (int v = 0; v < 4; ++v) part4[o][j][v] = src[(j * 4 + v) * 64 + lane];
          }
        }
        // Stage the 16 x 64 block (lane l: rows 4 (l / 16) + v of column
        // 16 j + l % 16), then write 16-byte row pieces.
        OutT* T = reinterpret_cast<OutT*>(outs + wave * 16 * kGOutPitch);
        constexpr int kTP = kGOutPitch * 4 / static_cast<int>(sizeof(OutT));  // staged row pitch, elements
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f32x4_t sum = (part4[0][j] + part4[1][j]) + (part4[2][j] + part4[3][j]);
#pragma unroll
          for (int v = 0; v < 4; ++v)
            T[(4 * (lane >> 4) + v) * kTP + 16 * j + (lane & 15)] = static_cast<OutT>(sum[v]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        constexpr int kPieces = 16 * 64 / kPer;
#pragma unroll
        for (int h2 = 0; h2 < kPieces / 64; ++h2) {
          const int c = lane + 64 * h2;
          const int r = c / (64 / kPer), col = (c % (64 / kPer)) * kPer;
          const int32_t pr = s_pair[16 * (hfb + q) + r];
          const int64_t gn = n0 + col;
          if (pr < 0 || gn >= n_rows) continue;
          OutT* dst = static_cast<OutT*>(y) + static_cast<int64_t>(pr) * n_rows + gn;
          const OutT* src = T + r * kTP + col;
          if (gn + kPer <= n_rows && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
            *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
          } else {
            for (int i2 = 0; i2 < kPer && gn + i2 < n_rows; ++i2) dst[i2] = src[i2];
          }
        }
      }
      __syncthreads();  // red and the staged rows are rewritten next
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  };

  // Unit u (d = u % 4): X of unit u + 3 into slot (d + 3) % 4; B operands of
  // MFMA group q from stage d; multiply; at even u, dequantize the pair of
  // units u + 2, u + 3 into stages (d + 2) % 4, (d + 3) % 4 from its ring
  // slot, which then takes the pieces of the pair two further on. Those
  // stages were last read at units u - 2 and u - 1 and are read next at
  // u + 2 and u + 3, so a barrier after every odd unit orders them.
  const auto unit = [&](int d) __attribute__((always_inline)) {
    prefetch(d);
    load_x(xa[(d + 3) & 3], cx);
    gadvance(cx, S);
    bf16x8_t bfr[4];
    const uint16_t* bs = Ws + d * kGStage + 32 * q + 8 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) bfr[j] = *reinterpret_cast<const bf16x8_t*>(bs + (16 * j + (lane & 15)) * kGPitch);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (i < mbn) {
        const bf16x8_t av = __builtin_bit_cast(bf16x8_t, xa[d].v[i]);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bfr[j], acc[i][j], 0, 0, 0);
      }
    }
    if ((d & 1) == 0) {
      // pair (u + 2) / 2: slot (d / 2 + 1) % 2, as u0 / 2 is even; units past
      // the last go to a stage no one reads (loads clamped to the last unit)
      MoePiece<TYPE>& pc = wr[((d >> 1) + 1) & 1];
      dequant(pc, (d + 2 + hh) & 3);
      load_w(pc, cw);
      adv2(cw);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (d & 1) __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    if (cc_.st == S - 1) epilogue(cc_.nt);
    gadvance(cc_, S);
  };

  for (int u0 = 0; u0 < U; u0 += 4) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      if (u0 + d < U) unit(d);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // the last prefetches
  asm volatile("" ::"v"(sink | pf[0] | pf[1] | pf[2] | pf[3]));
}

}  // namespace

// Whether the grouped-GEMM form takes this MUL_MAT_ID (the caller also needs
// a workspace of moe_gemm_workspace_bytes()).
bool moe_gemm_fits(int type, int64_t n_expert, int64_t n_pairs, int64_t k) {
  if (k <= 0 || k % 128 != 0 || k % block_elems(type) != 0) return false;
  if (n_expert <= 0 || n_expert > INT32_MAX / 2) return false;
  // the packed activations are addressed with 32-bit offsets
  const int64_t blocks = (n_pairs + 15 * n_expert) / 16 + 1;
  return blocks * 16 * k * 2 < (int64_t(1) << 31);
}

// Bytes the grouped-GEMM form needs after the routing lists: blk_base and
// mt_base (n_expert + 1 int32 each), then the packed activations.
int64_t moe_gemm_extra_bytes(int64_t n_expert, int64_t n_pairs, int64_t k) {
  const int64_t blocks = (n_pairs + 15 * n_expert) / 16 + 1;
  return 2 * 4 * (n_expert + 1) + 256 + blocks * 16 * k * 2;
}

// Packs the routed rows, then runs the grouped GEMM (arguments validated by
// the caller, moe_gemm_fits() holds, routing lists built).
int moe_gemm(int type, const void* w, int64_t expert_stride, int64_t n_expert, int64_t n_rows, int64_t k,
             const uint16_t* x, int64_t x_slots, int64_t top_k, int64_t n_pairs, const int32_t* offsets,
             const int32_t* list, const int32_t* blk_base, const int32_t* mt_base, void* xp_ws, void* y,
             int y_type, hipStream_t s) {
  uint16_t* xp = static_cast<uint16_t*>(xp_ws);
  const int64_t blocks = (n_pairs + 15 * n_expert) / 16 + 1;
  const uint32_t xp_bytes = static_cast<uint32_t>(blocks * 16 * k * 2);
  // Upper bound of the m-tiles (the kernel reads the exact count) and the
  // n-parts that give about one workgroup per CU.
  const int64_t mt_ub = std::min<int64_t>((n_pairs + (kGMTile - 1) * n_expert) / kGMTile + 1,
                                          ceil_div(n_pairs, kGMTile) + n_expert);
  const int64_t n_tiles = ceil_div(n_rows, kGBN);
  const int64_t mt_est = std::max<int64_t>(1, std::min(mt_ub, std::max(ceil_div(n_pairs, kGMTile), n_expert)));
  const int64_t parts = std::max<int64_t>(1, std::min(n_tiles, ceil_div(device_cu_count(), mt_est)));
  const int64_t grid = ceil_div(mt_ub, 8) * 8 * parts;
  const int64_t pack_x = std::max<int64_t>(1, std::min<int64_t>(64, ceil_div(4 * device_cu_count(), n_expert)));
  if (grid > INT32_MAX || n_expert > 65535) return SPIRAL_ERR_SHAPE;
#define SPIRAL_MOE_GEMM(T)                                                                                        \
  do {                                                                                                            \
    hipLaunchKernelGGL(moe_pack_kernel<T>, dim3(static_cast<unsigned>(pack_x), static_cast<unsigned>(n_expert)),  \
                       dim3(kGPackThreads), 0, s, x, k, x_slots, top_k, offsets, list, blk_base, xp);             \
    int rc = launch_status();                                                                                     \
    if (rc != SPIRAL_OK) return rc;                                                                               \
    if (y_type == SPIRAL_TYPE_F32)                                                                                \
      hipLaunchKernelGGL((moe_gemm_kernel<T, true>), dim3(static_cast<unsigned>(grid)), dim3(kGThreads), 0, s,    \
                         static_cast<const uint8_t*>(w), expert_stride, n_rows, k, xp, xp_bytes, offsets, list,   \
                         blk_base, mt_base, static_cast<int32_t>(n_expert), static_cast<int32_t>(parts), y);      \
    else                                                                                                          \
      hipLaunchKernelGGL((moe_gemm_kernel<T, false>), dim3(static_cast<unsigned>(grid)), dim3(kGThreads), 0, s,   \
                         static_cast<const uint8_t*>(w), expert_stride, n_rows, k, xp, xp_bytes, offsets, list,   \
                         blk_base, mt_base, static_cast<int32_t>(n_expert), static_cast<int32_t>(parts), y);      \
    return launch_status();                                                                                       \
  } while (0)
  switch (type) {
    case SPIRAL_TYPE_Q4_0: SPIRAL_MOE_GEMM(SPIRAL_TYPE_Q4_0);
    case SPIRAL_TYPE_Q8_0: SPIRAL_MOE_GEMM(SPIRAL_TYPE_Q8_0);
    case SPIRAL_TYPE_Q6_K: SPIRAL_MOE_GEMM(SPIRAL_TYPE_Q6_K);
    case SPIRAL_TYPE_Q4_K: SPIRAL_MOE_GEMM(SPIRAL_TYPE_Q4_K);
    case SPIRAL_TYPE_Q5_K: SPIRAL_MOE_GEMM(SPIRAL_TYPE_Q5_K);
    case SPIRAL_TYPE_IQ4_NL: SPIRAL_MOE_GEMM(SPIRAL_TYPE_IQ4_NL);
    case SPIRAL_TYPE_IQ4_XS: SPIRAL_MOE_GEMM(SPIRAL_TYPE_IQ4_XS);
    default: return SPIRAL_ERR_TYPE;
  }
#undef SPIRAL_MOE_GEMM
}

}  // namespace spiral
