// Grouped dequant-GEMM for mixture-of-experts (ggml MUL_MAT_ID with
// quantized, expert-stacked weights).
//
// Routing: at decode sizes (at most kFusedPairs (token, slot) pairs) each
// moe_kernel workgroup scans the ids for its own expert into LDS, and the
// workgroups of expert 0 also write the zero rows of pairs whose id is out
// of range: one launch. Larger batches first run route_kernel (one
// workgroup): a counting sort of the pairs by expert id into per-expert
// lists in the caller's workspace, pairs with an out-of-range id getting a
// zero output row.
//
// moe_stream_kernel (k <= kStreamMaxK, every shape the decode path meets):
//     a few workgroups per expert, each over a contiguous range of 16-row
//     groups; the routed tokens' activations are staged in LDS once and the
//     waves stream their weight rows with no barriers (see the streaming
//     section below).
//
// moe_kernel (larger k): workgroup (n-tile of 64 rows, expert) streams those weight
//     rows and multiplies them against the tokens routed to the expert, 16
//     tokens (one MFMA row block) per pass. At decode batch sizes (a few
//     tokens per expert) that is one pass, so each expert's weights are read
//     from HBM once per call, which is what bounds this op.
//
// moe_kernel layout (gfx950, v_mfma_f32_16x16x32_bf16):
//  - Wave w owns weight rows n0 + 16 w .. + 15 (the MFMA B columns). Lane l
//    serves row l % 16 and k-group g = l / 16. For every 128-wide k step it
//    takes one piece (Q4_0 / Q8_0: block 4 kb + g; Q6_K: 32-element group g
//    of the half super-block) and dequantizes it into the B operands of the
//    step's four MFMAs, so weights are never stored as bf16.
//  - The pieces come from LDS: pairs of k steps of the workgroup's 64 rows
//    are loaded with whole-line loads kStageAhead pairs ahead (register
//    ring) and written to one of two LDS stages (see WStage).
//  - An MFMA sums over its 32 k in any order as long as A and B agree; MFMA
//    s of a step takes, from lane group g, the 8 elements of piece g that
//    are cheapest to unpack (see MoePiece). The routed tokens' activations
//    are staged per kMoeKC-wide k chunk in LDS in exactly that order (only
//    the pass's real token rows; MFMA rows past them read a copy and their
//    outputs are dropped).
// Products use exactly dequantized bf16 weights and fp32 accumulation, as in
// the dense GEMM.
//
// GLU fused into the streaming form (ggml MUL_MAT_ID followed by GLU over
// its two halves, the merged gate/up FFN of MoE models): the expert matrix
// has 2F rows, gate rows [0, F) and up rows [F, 2F). Workgroups split the F
// output features; a wave streams feature group j's gate rows and then its
// up rows through the same register ring, keeps the gate sums, and writes
// act(gate) * up (act(up) * gate when swapped) to a [pair][F] output, so
// the [pair][2F] product never reaches memory. ggml's split form (gate and
// up experts in two tensors of F rows, two MUL_MAT_ID nodes and a GLU over
// both) runs the same way with the up rows taken from the second stack.
#include <algorithm>
#include <mutex>

#include "common.h"
#include "dequant_impl.h"
#include "moe_piece.h"

namespace spiral {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int kRouteThreads = 1024;
constexpr int kRouteChunk = 4096;  // experts counted per LDS pass
constexpr int kRouteLdsList = 8192;  // lists of up to this many pairs are built in LDS
constexpr int kMoeBN = 64;  // weight rows per workgroup (16 per wave)

// Workspace: offsets[n_expert + 1] then list[n_pairs] (int32).
//
// One workgroup: per chunk of kRouteChunk experts, count the pairs of each
// expert with LDS atomics, turn the counts into list offsets with a block
// scan, then scatter each pair's index into its expert's list. The order
// inside a list is arbitrary; each output row is computed on its own, so it
// does not change any result. Pairs with an id outside [0, n_expert) get a
// zero output row. Up to kRouteLdsList pairs, the scatter goes to LDS and the
// lists are written out contiguously at the end (scattered 4-byte stores
// from one CU were most of this kernel's time).
__global__ void __launch_bounds__(kRouteThreads) route_kernel(const int32_t* __restrict__ ids, int32_t n_pairs,
                                                              int32_t n_expert, int32_t* __restrict__ offsets,
                                                              int32_t* __restrict__ list, void* __restrict__ y,
                                                              int64_t out_cols, int y_f32) {
  __shared__ int32_t s_cnt[kRouteChunk];
  __shared__ int32_t s_wave[kRouteThreads / 64];
  __shared__ int32_t s_bad[kRouteThreads];
  __shared__ int32_t s_nbad;
  __shared__ int32_t s_list[kRouteLdsList];
  const bool lds_list = n_pairs <= kRouteLdsList;  // uniform
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  constexpr int kPer = kRouteChunk / kRouteThreads;
  // Each pass over the ids takes kRouteBatch of them per thread at a time,
  // every load issued before any is used: one load latency per batch
  // instead of one per id.
  constexpr int kRouteBatch = 8;
  if (tid == 0) s_nbad = 0;
  int32_t base = 0;
  for (int32_t e0 = 0; e0 < n_expert; e0 += kRouteChunk) {
    const int32_t ne = min(kRouteChunk, n_expert - e0);
    for (int i = tid; i < kRouteChunk; i += kRouteThreads) s_cnt[i] = 0;
    __syncthreads();
    // Count. The first chunk also collects the pairs routed nowhere (up to
    // kRouteThreads of them; s_nbad keeps counting past that).
    for (int32_t p0 = tid; p0 < n_pairs; p0 += kRouteBatch * kRouteThreads) {
      int32_t id[kRouteBatch];
#pragma unroll
      for (int u = 0; u < kRouteBatch; ++u) {
        const int32_t p = p0 + u * kRouteThreads;
        id[u] = p < n_pairs ? ids[p] : 0;
      }
#pragma unroll
      for (int u = 0; u < kRouteBatch; ++u) {
        const int32_t p = p0 + u * kRouteThreads;
        if (p >= n_pairs) break;
        if (id[u] >= e0 && id[u] < e0 + ne) atomicAdd(&s_cnt[id[u] - e0], 1);
        if (e0 == 0 && (id[u] < 0 || id[u] >= n_expert)) {
          const int32_t b = atomicAdd(&s_nbad, 1);
          if (b < kRouteThreads) s_bad[b] = p;
        }
      }
    }
    __syncthreads();
    // Exclusive scan: thread t owns experts [kPer t, kPer t + kPer).
    int32_t c[kPer], run = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      c[i] = s_cnt[kPer * tid + i];
      run += c[i];
    }
    int32_t incl = run;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int32_t v = __shfl_up(incl, off, 64);
      if (lane >= off) incl += v;
    }
    if (lane == 63) s_wave[wv] = incl;
    __syncthreads();
    int32_t wbase = 0, total = 0;
    for (int i = 0; i < kRouteThreads / 64; ++i) {
      const int32_t v = s_wave[i];
      wbase += i < wv ? v : 0;
      total += v;
    }
    int32_t pos = base + wbase + incl - run;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int e = kPer * tid + i;
      if (e < ne) offsets[e0 + e] = pos;
      s_cnt[e] = pos;
      pos += c[i];
    }
    __syncthreads();
    // Scatter each pair's index into its expert's list.
    for (int32_t p0 = tid; p0 < n_pairs; p0 += kRouteBatch * kRouteThreads) {
      int32_t id[kRouteBatch];
#pragma unroll
      for (int u = 0; u < kRouteBatch; ++u) {
        const int32_t p = p0 + u * kRouteThreads;
        id[u] = p < n_pairs ? ids[p] : -1;
      }
#pragma unroll
      for (int u = 0; u < kRouteBatch; ++u) {
        const int32_t p = p0 + u * kRouteThreads;
        if (p >= n_pairs) break;
        if (id[u] >= e0 && id[u] < e0 + ne) {
          const int32_t q = atomicAdd(&s_cnt[id[u] - e0], 1);
          if (lds_list)
            s_list[q] = p;
          else
            list[q] = p;
        }
      }
    }
    base += total;
    __syncthreads();
  }
  if (tid == 0) offsets[n_expert] = base;
  if (lds_list) {  // positions [0, base) were all written (the loop ended with a barrier)
    for (int32_t i = tid; i < base; i += kRouteThreads) list[i] = s_list[i];
  }
  // Pairs routed nowhere produce a zero row, cleared by the whole workgroup.
  const auto clear_row = [&](int64_t row) {
    for (int64_t col = tid; col < out_cols; col += kRouteThreads) {
      if (y_f32)
        static_cast<float*>(y)[row * out_cols + col] = 0.0f;
      else
        static_cast<uint16_t*>(y)[row * out_cols + col] = 0;
    }
  };
  const int32_t nbad = s_nbad;  // final: the chunk loop (n_expert >= 1) ended with a barrier
  if (nbad <= kRouteThreads) {
    for (int32_t b = 0; b < nbad; ++b) clear_row(s_bad[b]);
    return;
  }
  // More than kRouteThreads of them: collect and clear kRouteThreads at a time.
  for (int32_t p0 = 0; p0 < n_pairs; p0 += kRouteThreads) {
    __syncthreads();
    if (tid == 0) s_nbad = 0;
    __syncthreads();
    const int32_t p = p0 + tid;
    if (p < n_pairs) {
      const int32_t e = ids[p];
      if (e < 0 || e >= n_expert) s_bad[atomicAdd(&s_nbad, 1)] = p;
    }
    __syncthreads();
    const int32_t nb = s_nbad;
    for (int32_t b = 0; b < nb; ++b) clear_row(s_bad[b]);
  }
}


constexpr int kMoeKC = 768;                   // k chunk of activations staged in LDS (3 pairs)
constexpr int kMoeTok = 16;                   // tokens per pass (one MFMA row block)
// Staged activation rows are padded by kAPad bf16 (64 bytes): an MFMA A
// read has lane (row r, group g) at byte 64 s + 16 g of row r, so a row
// offset of 64 bytes puts the 16 (r mod 4, g) starts on 16 different groups
// of 4 banks (a 16-byte pad would put rows r and r + 1 on the banks of
// groups g and g + 1).
constexpr int kAPad = 32;
constexpr int kMoeAPitch = kMoeKC + kAPad;    // bf16 per staged row
constexpr int kFusedPairs = 1024;             // largest batch routed inside moe_kernel
constexpr int kMaxRouteWaves = 16;            // waves of a routing workgroup (at most 1024 threads)
constexpr int kStageAhead = 3;                // weight pairs in flight in registers
static_assert(kMoeKC % 256 == 0, "activation chunks hold whole weight pairs");

// ---- weights staged through LDS -------------------------------------------
//
// A stage is one pair of 128-wide k steps (256 k) of the workgroup's 64
// weight rows. Each thread loads its share with whole-line loads (8 or 16
// lanes per 128-byte line of a row) into registers kStageAhead pairs ahead,
// writes it to an LDS stage, and each wave then reads its MFMA pieces (16
// rows x 4 lane groups) from LDS. Loading the pieces directly would touch
// 16 rows per instruction, 16 or 2 bytes of each. Offsets are 32-bit (the
// launcher keeps each expert matrix below 2 GiB); rows past n_rows are
// clamped (their outputs are never stored) and blocks past k read as zero.
template <int TYPE>
struct WStage;

// Q4_0 pair: per row 8 blocks, qs 128 bytes (LDS pitch 144) and d 16 bytes.
template <>
struct WStage<SPIRAL_TYPE_Q4_0> {
  static constexpr int kQsPitch = 144, kDOff = 64 * kQsPitch, kBytes = kDOff + 64 * 16;
  struct Addr {
    uint32_t q[2], d;
    int qc, dc;
  };
  uint4 q[2];
  uint32_t d0, d1;
  // thread t: qs of rows 32 i + t / 8 (i < 2), block t % 8; d of row t / 4,
  // blocks 2 (t % 4) and 2 (t % 4) + 1.
  static __device__ __forceinline__ Addr addr(int64_t n0, int64_t n_rows, int64_t nb, int t) {
    Addr a;
    for (int i = 0; i < 2; ++i)
      a.q[i] = static_cast<uint32_t>((min(n0 + 32 * i + t / 8, n_rows - 1) * nb + t % 8) * 16);
    a.qc = t % 8;
    a.dc = 2 * (t % 4);
    a.d = static_cast<uint32_t>((min(n0 + t / 4, n_rows - 1) * nb + a.dc) * 2);
    return a;
  }
  __device__ __forceinline__ void load(const Planes& P, const Addr& a, int64_t p, int64_t nb) {
    const int64_t b = 8 * p;
    const uint32_t sq = static_cast<uint32_t>(b * 16), sd = static_cast<uint32_t>(b * 2);
    const bool qv = b + a.qc < nb;
    for (int i = 0; i < 2; ++i) q[i] = qv ? bload16(P.a, a.q[i], sq) : make_uint4(0u, 0u, 0u, 0u);
    d0 = b + a.dc < nb ? bload2(P.d, a.d, sd) : 0u;
    d1 = b + a.dc + 1 < nb ? bload2(P.d, a.d + 2, sd) : 0u;
  }
  __device__ __forceinline__ void store(uint8_t* st, int t) const {
    for (int i = 0; i < 2; ++i) *reinterpret_cast<uint4*>(st + (32 * i + t / 8) * kQsPitch + (t % 8) * 16) = q[i];
    *reinterpret_cast<uint32_t*>(st + kDOff + (t / 4) * 16 + (t % 4) * 4) = d0 | (d1 << 16);
  }
  // Piece of row r (0..63) for step h (0, 1) of the pair and lane group g.
  static __device__ __forceinline__ void piece(MoePiece<SPIRAL_TYPE_Q4_0>& pc, const uint8_t* st, int r, int h, int g) {
    pc.q = *reinterpret_cast<const uint4*>(st + r * kQsPitch + (4 * h + g) * 16);
    pc.d = *reinterpret_cast<const uint16_t*>(st + kDOff + r * 16 + (4 * h + g) * 2);
  }
};

// Q8_0 pair: per row 8 blocks, qs 256 bytes (LDS pitch 272) and d 16 bytes.
template <>
struct WStage<SPIRAL_TYPE_Q8_0> {
  static constexpr int kQsPitch = 272, kDOff = 64 * kQsPitch, kBytes = kDOff + 64 * 16;
  struct Addr {
    uint32_t q[4], d;
    int qc, dc;
  };
  uint4 q[4];
  uint32_t d0, d1;
  // thread t: qs bytes 16 (t % 16) .. + 15 of rows 16 i + t / 16 (i < 4).
  static __device__ __forceinline__ Addr addr(int64_t n0, int64_t n_rows, int64_t nb, int t) {
    Addr a;
    for (int i = 0; i < 4; ++i)
      a.q[i] = static_cast<uint32_t>(min(n0 + 16 * i + t / 16, n_rows - 1) * nb * 32 + (t % 16) * 16);
    a.qc = (t % 16) / 2;
    a.dc = 2 * (t % 4);
    a.d = static_cast<uint32_t>((min(n0 + t / 4, n_rows - 1) * nb + a.dc) * 2);
    return a;
  }
  __device__ __forceinline__ void load(const Planes& P, const Addr& a, int64_t p, int64_t nb) {
    const int64_t b = 8 * p;
    const uint32_t sq = static_cast<uint32_t>(b * 32), sd = static_cast<uint32_t>(b * 2);
    const bool qv = b + a.qc < nb;
    for (int i = 0; i < 4; ++i) q[i] = qv ? bload16(P.a, a.q[i], sq) : make_uint4(0u, 0u, 0u, 0u);
    d0 = b + a.dc < nb ? bload2(P.d, a.d, sd) : 0u;
    d1 = b + a.dc + 1 < nb ? bload2(P.d, a.d + 2, sd) : 0u;
  }
  __device__ __forceinline__ void store(uint8_t* st, int t) const {
    for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(st + (16 * i + t / 16) * kQsPitch + (t % 16) * 16) = q[i];
    *reinterpret_cast<uint32_t*>(st + kDOff + (t / 4) * 16 + (t % 4) * 4) = d0 | (d1 << 16);
  }
  static __device__ __forceinline__ void piece(MoePiece<SPIRAL_TYPE_Q8_0>& pc, const uint8_t* st, int r, int h, int g) {
    pc.q0 = *reinterpret_cast<const uint4*>(st + r * kQsPitch + (4 * h + g) * 32);
    pc.q1 = *reinterpret_cast<const uint4*>(st + r * kQsPitch + (4 * h + g) * 32 + 16);
    pc.d = *reinterpret_cast<const uint16_t*>(st + kDOff + r * 16 + (4 * h + g) * 2);
  }
};

// Q6_K pair: one super-block per row: ql 128 bytes (pitch 144), qh 64 (pitch
// 80), sc 16, d 2.
template <>
struct WStage<SPIRAL_TYPE_Q6_K> {
  static constexpr int kQhOff = 64 * 144, kScOff = kQhOff + 64 * 80, kDOff = kScOff + 64 * 16, kBytes = kDOff + 64 * 2;
  struct Addr {
    uint32_t l[2], h, sc, d;
  };
  uint4 l[2], h;
  uint32_t sc, d;
  // thread t: ql bytes 16 (t % 8) of rows 32 i + t / 8; qh bytes 16 (t % 4)
  // and sc bytes 4 (t % 4) of row t / 4; d of row t (t < 64).
  static __device__ __forceinline__ Addr addr(int64_t n0, int64_t n_rows, int64_t nb, int t) {
    Addr a;
    for (int i = 0; i < 2; ++i)
      a.l[i] = static_cast<uint32_t>(min(n0 + 32 * i + t / 8, n_rows - 1) * nb * 128 + (t % 8) * 16);
    const int64_t r4 = min(n0 + t / 4, n_rows - 1) * nb;
    a.h = static_cast<uint32_t>(r4 * 64 + (t % 4) * 16);
    a.sc = static_cast<uint32_t>(r4 * 16 + (t % 4) * 4);
    a.d = static_cast<uint32_t>(min(n0 + (t & 63), n_rows - 1) * nb * 2);
    return a;
  }
  __device__ __forceinline__ void load(const Planes& P, const Addr& a, int64_t p, int64_t) {
    const uint32_t sb = static_cast<uint32_t>(p);
    for (int i = 0; i < 2; ++i) l[i] = bload16(P.a, a.l[i], sb * 128u);
    h = bload16(P.b, a.h, sb * 64u);
    const auto v = __builtin_amdgcn_raw_buffer_load_b32(P.c, a.sc, sb * 16u, 0);
    sc = static_cast<uint32_t>(v);
    d = bload2(P.d, a.d, sb * 2u);
  }
  __device__ __forceinline__ void store(uint8_t* st, int t) const {
    for (int i = 0; i < 2; ++i) *reinterpret_cast<uint4*>(st + (32 * i + t / 8) * 144 + (t % 8) * 16) = l[i];
    *reinterpret_cast<uint4*>(st + kQhOff + (t / 4) * 80 + (t % 4) * 16) = h;
    *reinterpret_cast<uint32_t*>(st + kScOff + (t / 4) * 16 + (t % 4) * 4) = sc;
    if (t < 64) *reinterpret_cast<uint16_t*>(st + kDOff + t * 2) = static_cast<uint16_t>(d);
  }
  static __device__ __forceinline__ void piece(MoePiece<SPIRAL_TYPE_Q6_K>& pc, const uint8_t* st, int r, int h, int g) {
    const uint8_t* ql = st + r * 144 + 64 * h + 32 * (g & 1);
    const uint8_t* qh = st + kQhOff + r * 80 + 32 * h;
    pc.l0 = *reinterpret_cast<const uint4*>(ql);
    pc.l1 = *reinterpret_cast<const uint4*>(ql + 16);
    pc.h0 = *reinterpret_cast<const uint4*>(qh);
    pc.h1 = *reinterpret_cast<const uint4*>(qh + 16);
    const uint32_t sc = *reinterpret_cast<const uint16_t*>(st + kScOff + r * 16 + 8 * h + 2 * g);
    pc.ds2 = *reinterpret_cast<const uint16_t*>(st + kDOff + r * 2) | (sc << 16);
    pc.sch = 0u;
    pc.ls = (g >> 1) * 4;
    pc.hs = 2 * g;
  }
};

// Q4_K / Q5_K pair: one super-block per row: qs 128 bytes (pitch 144), qh 32
// (Q5_K, pitch 48), meta 16.
template <int TYPE>
struct WStageKQ {
  static constexpr bool kQ5 = TYPE == SPIRAL_TYPE_Q5_K;
  static constexpr int kQhOff = 64 * 144, kMetaOff = kQhOff + (kQ5 ? 64 * 48 : 0), kBytes = kMetaOff + 64 * 16;
  struct Addr {
    uint32_t q[2], qh, meta;
  };
  uint4 q[2];
  uint32_t meta, h0, h1;
  // thread t: qs bytes 16 (t % 8) of rows 32 i + t / 8; meta dword t % 4 and
  // qh bytes 8 (t % 4) .. + 7 of row t / 4.
  static __device__ __forceinline__ Addr addr(int64_t n0, int64_t n_rows, int64_t nb, int t) {
    Addr a;
    for (int i = 0; i < 2; ++i)
      a.q[i] = static_cast<uint32_t>(min(n0 + 32 * i + t / 8, n_rows - 1) * nb * 128 + (t % 8) * 16);
    const int64_t r4 = min(n0 + t / 4, n_rows - 1) * nb;
    a.qh = static_cast<uint32_t>(r4 * 32 + (t % 4) * 8);
    a.meta = static_cast<uint32_t>(r4 * 16 + (t % 4) * 4);
    return a;
  }
  __device__ __forceinline__ void load(const Planes& P, const Addr& a, int64_t p, int64_t) {
    const uint32_t sb = static_cast<uint32_t>(p);
    for (int i = 0; i < 2; ++i) q[i] = bload16(P.a, a.q[i], sb * 128u);
    meta = bload4(P.c, a.meta, sb * 16u);
    if constexpr (kQ5) {
      h0 = bload4(P.b, a.qh, sb * 32u);
      h1 = bload4(P.b, a.qh + 4u, sb * 32u);
    }
  }
  __device__ __forceinline__ void store(uint8_t* st, int t) const {
    for (int i = 0; i < 2; ++i) *reinterpret_cast<uint4*>(st + (32 * i + t / 8) * 144 + (t % 8) * 16) = q[i];
    *reinterpret_cast<uint32_t*>(st + kMetaOff + (t / 4) * 16 + (t % 4) * 4) = meta;
    if constexpr (kQ5) *reinterpret_cast<uint2*>(st + kQhOff + (t / 4) * 48 + (t % 4) * 8) = make_uint2(h0, h1);
  }
  static __device__ __forceinline__ void piece(MoePiece<TYPE>& pc, const uint8_t* st, int r, int h, int g) {
    pc.q = *reinterpret_cast<const uint4*>(st + r * 144 + 64 * h + 32 * (g >> 1) + 16 * (g & 1));
    pc.meta = *reinterpret_cast<const uint4*>(st + kMetaOff + r * 16);
    if constexpr (kQ5) pc.qh = *reinterpret_cast<const uint4*>(st + kQhOff + r * 48 + 16 * (g & 1));
    pc.grp = 4 * h + 2 * (g >> 1);
  }
};
template <>
struct WStage<SPIRAL_TYPE_Q4_K> : WStageKQ<SPIRAL_TYPE_Q4_K> {};
template <>
struct WStage<SPIRAL_TYPE_Q5_K> : WStageKQ<SPIRAL_TYPE_Q5_K> {};

// IQ4_NL pair: Q4_0's staging (the planar layouts match).
template <>
struct WStage<SPIRAL_TYPE_IQ4_NL> : WStage<SPIRAL_TYPE_Q4_0> {
  static __device__ __forceinline__ void piece(MoePiece<SPIRAL_TYPE_IQ4_NL>& pc, const uint8_t* st, int r, int h, int g) {
    pc.q = *reinterpret_cast<const uint4*>(st + r * kQsPitch + (4 * h + g) * 16);
    pc.meta = make_uint2(*reinterpret_cast<const uint16_t*>(st + kDOff + r * 16 + (4 * h + g) * 2), 0u);
    pc.sub = 0;
  }
};

// IQ4_XS pair: one super-block per row: qs 128 bytes (pitch 144) and meta 8.
template <>
struct WStage<SPIRAL_TYPE_IQ4_XS> {
  static constexpr int kMetaOff = 64 * 144, kBytes = kMetaOff + 64 * 8;
  struct Addr {
    uint32_t q[2], meta;
  };
  uint4 q[2];
  uint32_t meta;
  // thread t: qs bytes 16 (t % 8) of rows 32 i + t / 8; meta dword t % 2 of
  // row t / 4 (t % 4 >= 2 repeat it).
  static __device__ __forceinline__ Addr addr(int64_t n0, int64_t n_rows, int64_t nb, int t) {
    Addr a;
    for (int i = 0; i < 2; ++i)
      a.q[i] = static_cast<uint32_t>(min(n0 + 32 * i + t / 8, n_rows - 1) * nb * 128 + (t % 8) * 16);
    a.meta = static_cast<uint32_t>(min(n0 + t / 4, n_rows - 1) * nb * 8 + (t % 2) * 4);
    return a;
  }
  __device__ __forceinline__ void load(const Planes& P, const Addr& a, int64_t p, int64_t) {
    const uint32_t sb = static_cast<uint32_t>(p);
    for (int i = 0; i < 2; ++i) q[i] = bload16(P.a, a.q[i], sb * 128u);
    meta = bload4(P.c, a.meta, sb * 8u);
  }
  __device__ __forceinline__ void store(uint8_t* st, int t) const {
    for (int i = 0; i < 2; ++i) *reinterpret_cast<uint4*>(st + (32 * i + t / 8) * 144 + (t % 8) * 16) = q[i];
    if ((t % 4) < 2) *reinterpret_cast<uint32_t*>(st + kMetaOff + (t / 4) * 8 + (t % 2) * 4) = meta;
  }
  static __device__ __forceinline__ void piece(MoePiece<SPIRAL_TYPE_IQ4_XS>& pc, const uint8_t* st, int r, int h, int g) {
    pc.q = *reinterpret_cast<const uint4*>(st + r * 144 + 64 * h + 16 * g);
    pc.meta = *reinterpret_cast<const uint2*>(st + kMetaOff + r * 8);
    pc.sub = 4 * h + g;
  }
};

// Stage activations k in [c0, c0 + kMoeKC) of the pass's nt token rows in
// MFMA order: item = 8 consecutive LDS positions (one lane group of one MFMA)
// of one row. Positions past k are zero.
template <int TYPE>
__device__ __forceinline__ void moe_stage(uint16_t* As, const uint16_t* __restrict__ x, const int64_t* xrow, int nt,
                                          int64_t k, int64_t c0, int tid, int width = kMoeKC, int pitch = kMoeAPitch,
                                          int nthreads = 256) {
  // Items go to threads kStageBatch at a time, every load of a batch issued
  // before any is stored, so a thread waits once per batch for the gathered
  // rows instead of once per item.
  constexpr int kStageBatch = 4;
  const int kItems = width / 8, total = nt * kItems;
  for (int it0 = tid; it0 < total; it0 += kStageBatch * nthreads) {
    uint2 lo[kStageBatch], hi[kStageBatch];
#pragma unroll
    for (int b = 0; b < kStageBatch; ++b) {
      const int it = it0 + b * nthreads;
      lo[b] = hi[b] = make_uint2(0u, 0u);
      if (it < total) {
        const int r = it / kItems, q = it % kItems;
        const int j = q >> 4, s = (q >> 2) & 3, gg = q & 3;
        const int64_t kb = c0 + 128 * j;
        const uint16_t* src = x + xrow[r] + kb;
        const int k0 = MoePiece<TYPE>::local(gg, s, 0), k4 = MoePiece<TYPE>::local(gg, s, 4);
        if (kb + k0 < k) lo[b] = *reinterpret_cast<const uint2*>(src + k0);
        if (kb + k4 < k) hi[b] = *reinterpret_cast<const uint2*>(src + k4);
      }
      if constexpr (kStageSwap<TYPE>) {
        lo[b] = stage_swap(lo[b]);
        hi[b] = stage_swap(hi[b]);
      }
    }
#pragma unroll
    for (int b = 0; b < kStageBatch; ++b) {
      const int it = it0 + b * nthreads;
      if (it < total) {
        const int r = it / kItems, q = it % kItems;
        *reinterpret_cast<uint4*>(&As[r * pitch + 8 * q]) = make_uint4(lo[b].x, lo[b].y, hi[b].x, hi[b].y);
      }
    }
  }
}

// offsets == nullptr: fused routing (n_pairs <= kFusedPairs) from ids;
// otherwise the expert's pairs are list[offsets[e] .. offsets[e + 1]).
template <int TYPE, bool F32_OUT>
__global__ void __launch_bounds__(256) moe_kernel(const uint8_t* __restrict__ w, int64_t expert_stride,
                                                  int64_t n_rows, int64_t k, const uint16_t* __restrict__ x,
                                                  int64_t x_slots, int64_t top_k, const int32_t* __restrict__ ids,
                                                  int32_t n_pairs, int32_t n_expert,
                                                  const int32_t* __restrict__ offsets,
                                                  const int32_t* __restrict__ list, void* __restrict__ y) {
  __shared__ __align__(16) uint16_t As[kMoeTok * kMoeAPitch];
  __shared__ __align__(16) uint8_t Ws[2 * WStage<TYPE>::kBytes];
  __shared__ int32_t s_pair[kMoeTok];
  __shared__ int64_t s_xrow[kMoeTok];
  __shared__ int32_t s_list[kFusedPairs];
  __shared__ int32_t s_n;
  const int64_t e = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  int32_t begin, end;
  const int32_t* lst;
  if (offsets == nullptr) {
    // Fused routing: the pairs routed to e, in any order (each output row is
    // computed on its own). Expert 0's workgroups also clear the rows of
    // pairs routed nowhere, each over its own 64 columns.
    if (tid == 0) s_n = 0;
    __syncthreads();
    for (int32_t p = tid; p < n_pairs; p += 256) {
      const int32_t id = ids[p];
      if (id == e) s_list[atomicAdd(&s_n, 1)] = p;
      if (e == 0 && (id < 0 || id >= n_expert)) {
        const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kMoeBN;
        for (int64_t c = c0; c < min(c0 + kMoeBN, n_rows); ++c) {
          if constexpr (F32_OUT)
            static_cast<float*>(y)[p * n_rows + c] = 0.0f;
          else
            static_cast<uint16_t*>(y)[p * n_rows + c] = 0;
        }
      }
    }
    __syncthreads();
    begin = 0;
    end = s_n;
    lst = s_list;
  } else {
    begin = offsets[e];
    end = offsets[e + 1];
    lst = list;
  }
  if (begin >= end) return;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kMoeBN;
  const int64_t n = n0 + 16 * wave + (lane & 15);  // this lane's weight row (MFMA column)
  const int r = 16 * wave + (lane & 15);            // its row within the stage
  const int64_t nb = k / block_elems(TYPE);
  const int64_t steps = (k + 127) / 128, pairs = (steps + 1) / 2;
  constexpr int kPairsPerChunk = kMoeKC / 256;
  const Planes P = make_planes<TYPE>(w + e * expert_stride, n_rows, nb);
  const typename WStage<TYPE>::Addr wa = WStage<TYPE>::addr(n0, n_rows, nb, tid);

  for (int32_t t0 = begin; t0 < end; t0 += kMoeTok) {
    const int nt = min(kMoeTok, end - t0);
    __syncthreads();
    if (tid < kMoeTok) {
      const int32_t pr = tid < nt ? lst[t0 + tid] : -1;
      s_pair[tid] = pr;
      if (pr >= 0) {
        const int64_t t = pr / top_k, slot = pr % top_k;
        s_xrow[tid] = (t * x_slots + slot % x_slots) * k;
      }
    }
    // Weights do not depend on the tokens: start the ring first.
    WStage<TYPE> ring[kStageAhead];
#pragma unroll
    for (int i = 0; i < kStageAhead; ++i) ring[i].load(P, wa, min<int64_t>(i, pairs - 1), nb);
    __syncthreads();
    // MFMA rows past nt read row nt - 1; their outputs are dropped.
    const uint16_t* arow = As + min(lane & 15, nt - 1) * kMoeAPitch + 8 * g;
    // One accumulator per MFMA of a step, so consecutive MFMAs do not wait
    // for each other's results; summed at the end.
    f32x4_t acc[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) acc[s] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    moe_stage<TYPE>(As, x, s_xrow, nt, k, 0, tid);
    ring[0].store(Ws, tid);
    ring[0].load(P, wa, min<int64_t>(kStageAhead, pairs - 1), nb);
    __syncthreads();

    // Pair p sits in LDS stage p % 2 and, before that, in ring slot
    // p % kStageAhead. One barrier per pair orders both LDS buffers. A chunk
    // of activations holds kStageAhead pairs, so inside it the ring slot and
    // the activation offsets are compile-time constants.
    static_assert(kStageAhead == kPairsPerChunk, "ring slots follow the pair index inside a chunk");
    const int64_t chunks = (pairs + kPairsPerChunk - 1) / kPairsPerChunk;
    for (int64_t c = 0; c < chunks; ++c) {
      if (c > 0) {
        moe_stage<TYPE>(As, x, s_xrow, nt, k, c * kMoeKC, tid);
        __syncthreads();
      }
#pragma unroll
      for (int d = 0; d < kPairsPerChunk; ++d) {
        const int64_t p = c * kPairsPerChunk + d;
        if (p >= pairs) break;
        const uint8_t* st = Ws + (p & 1) * WStage<TYPE>::kBytes;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (h == 0 || 2 * p + 1 < steps) {
            MoePiece<TYPE> pc;
            WStage<TYPE>::piece(pc, st, r, h, g);
            pc.prep();
#pragma unroll
            for (int s = 0; s < 4; ++s) {
              const bf16x8_t b = __builtin_bit_cast(bf16x8_t, pc.dequant(s));
              const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(arow + 8 * (16 * (2 * d + h) + 4 * s));
              acc[s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[s], 0, 0, 0);
            }
          }
        }
        if (p + 1 < pairs) {
          ring[(d + 1) % kStageAhead].store(Ws + ((p + 1) & 1) * WStage<TYPE>::kBytes, tid);
          ring[(d + 1) % kStageAhead].load(P, wa, min<int64_t>(p + 1 + kStageAhead, pairs - 1), nb);
        }
        __syncthreads();
      }
    }

    // acc: lane l holds rows 4 (l / 16) + i (routed pairs) of column l % 16
    // (weight row n).
    const f32x4_t sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int32_t pr = s_pair[4 * g + i];
      if (pr >= 0 && n < n_rows) {
        if constexpr (F32_OUT)
          static_cast<float*>(y)[pr * n_rows + n] = sum[i];
        else
          static_cast<__bf16*>(y)[pr * n_rows + n] = static_cast<__bf16>(sum[i]);
      }
    }
  }
}


// ---- GLU activations (ggml GLU ops, fp32) -----------------------------------
// act(a) * b for the ggml GLU variants (ids as in include/spiral_ggml.h):
// REGLU relu, GEGLU gelu (tanh form), SWIGLU silu, GEGLU_ERF gelu (erf form),
// GEGLU_QUICK x * sigmoid(1.702 x).
__device__ __forceinline__ float glu_act(int op, float a) {
  switch (op) {
    case SPIRAL_GLU_REGLU: return a > 0.0f ? a : 0.0f;
    case SPIRAL_GLU_GEGLU: {
      const float u = 0.7978845608028654f * a * (1.0f + 0.044715f * a * a);  // sqrt(2/pi) (a + 0.044715 a^3)
      return 0.5f * a * (1.0f + tanhf(u));
    }
    case SPIRAL_GLU_SWIGLU: return a / (1.0f + expf(-a));
    case SPIRAL_GLU_GEGLU_ERF: return 0.5f * a * (1.0f + erff(a * 0.7071067811865476f));
    default: return a / (1.0f + expf(-1.702f * a));  // SPIRAL_GLU_GEGLU_QUICK
  }
}

// One output of a standalone GLU: act(a) * b, a the activated half. SWIGLU_OAI
// (gpt-oss, as ggml computes it): with x = min(a, limit) and
// y = clamp(b, -limit, limit), x / (1 + exp(-alpha x)) * (y + 1); min and
// clamp written as comparisons, as std::min and std::clamp evaluate them.
__device__ __forceinline__ float glu_pair(int op, float a, float b, float alpha, float limit) {
  if (op == SPIRAL_GLU_SWIGLU_OAI) {
    const float x = limit < a ? limit : a;
    const float y = b < -limit ? -limit : (limit < b ? limit : b);
    return x / (1.0f + expf(alpha * (-x))) * (y + 1.0f);
  }
  return glu_act(op, a) * b;
}

// Standalone ggml GLU over rows of 2n floats: y[r][i] = act(h0[i]) * h1[i]
// with (h0, h1) = (x[r][0 .. n), x[r][n .. 2n)), swapped: the other order.
__global__ void __launch_bounds__(256) glu_kernel(const float* __restrict__ x, int64_t ldx, float* __restrict__ y,
                                                  int64_t ldy, int64_t n, int64_t rows, int op, int swapped,
                                                  float alpha, float limit) {
  const int64_t total = n * rows;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t r = i / n, c = i - r * n;
    const float* xr = x + r * ldx;
    const float a = xr[swapped ? c + n : c], b = xr[swapped ? c : c + n];
    y[r * ldy + c] = glu_pair(op, a, b, alpha, limit);
  }
}

// ggml's split form: gate and up rows in two tensors; y = act(gate) * up
// (act(up) * gate when swapped).
__global__ void __launch_bounds__(256) glu_split_kernel(const float* __restrict__ xg, int64_t ldg,
                                                        const float* __restrict__ xu, int64_t ldu,
                                                        float* __restrict__ y, int64_t ldy, int64_t n, int64_t rows,
                                                        int op, int swapped, float alpha, float limit) {
  const int64_t total = n * rows;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t r = i / n, c = i - r * n;
    const float g = xg[r * ldg + c], u = xu[r * ldu + c];
    y[r * ldy + c] = swapped ? glu_pair(op, u, g, alpha, limit) : glu_pair(op, g, u, alpha, limit);
  }
}

// ---- streaming form (the decode path) ------------------------------------
//
// When the activations of 16 tokens over the whole k fit in LDS (k <= 4096)
// the workgroup stages them once per pass of 16 tokens and its waves then run
// without barriers: wave w takes the 16-row groups w, w + 8, ... of the
// workgroup's row range and streams (group, k step) items end to end through
// its own register ring of pieces, loaded straight from memory with buffer
// loads. A few workgroups per expert (about two per CU in total) each cover a
// contiguous range of rows, so the routing scan and the activation staging
// are paid a few hundred times per call instead of once per 64 rows.
// Waves per workgroup of the streaming form. Prefill passes (TB >= 2) stage
// up to 128 KiB of activations, so one workgroup fits a CU: 12 waves (three
// a SIMD, as their registers allow) share that staging instead of 8. The
// fused GLU form and Q6_K at four row blocks need more registers than three
// waves a SIMD leave them.
template <int TYPE, bool GLU, int TB>
constexpr int kStreamWaves = (TB >= 2 && !GLU && !(TYPE == SPIRAL_TYPE_Q6_K && TB == 4)) ? 12 : 8;
constexpr int64_t kStreamMaxK = 4096;

// Waves per SIMD the compiler must leave room for (launch bounds). Decode
// passes (TB = 1, 8-wave workgroups) are held to four, so two workgroups
// share a CU (their staged rows fit its LDS twice): the Q4_0 fused GLU form
// would otherwise take 130 registers and fit one. Q6_K would spill there.
template <int TYPE, int TB, int WAVES>
constexpr int kStreamMinWaves = (TB == 1 && WAVES == 8 && TYPE != SPIRAL_TYPE_Q6_K) ? 4 : 1;

// Ring slots (units) in flight per wave.
template <int TYPE>
constexpr int kStreamRing = TYPE == SPIRAL_TYPE_Q4_0 ? 4 : TYPE == SPIRAL_TYPE_Q8_0 ? 6 : 4;


// What one ring slot of the streaming form holds (a "unit"), loaded for one
// 16-row group of the wave. Q4_0: a pair of k steps of all 16 rows, loaded
// as whole 128-byte lines (two instructions, rows 0..7 and 8..15) and moved
// into MFMA position with ds_bpermute; loading the pieces directly would
// fetch every line as two 64-byte halves, which the L1's miss capacity turns
// into the limit. After arrange(), one register holds step h of the pair
// for all 16 rows, and each permute reads every one of its 64 source lanes
// once.
// Other types: one k step's pieces, loaded directly.
template <int TYPE>
struct Unit {
  static constexpr int kSteps = 1;
  MoePiece<TYPE> pc;
  struct Addr {
    PieceAddr<TYPE> pa;
  };
  static __device__ __forceinline__ Addr addr(int64_t row0, int64_t n_rows, int64_t nb, int lane) {
    Addr a;
    a.pa.set(min(row0 + (lane & 15), n_rows - 1), nb, lane >> 4);
    return a;
  }
  __device__ __forceinline__ void load(const Planes& P, const Addr& a, int64_t u, int64_t) { a.pa.load(pc, P, u); }
  __device__ __forceinline__ void arrange() {}
  __device__ __forceinline__ void piece(MoePiece<TYPE>& out, int, int) const { out = pc; }
};

template <>
struct Unit<SPIRAL_TYPE_Q4_0> {
  static constexpr int kSteps = 2;
  // As loaded, lane l = 32 h + 4 r' + c': qa / qb hold rows r' and 8 + r'
  // of the group, block 8 u + 4 h + c' (arrange() regroups them by step).
  // d0 / d1 are already in MFMA lane order: lane (r, g) = (l % 16, l / 16)
  // holds the dword that contains the fp16 d of block 8 u + g (d0) and
  // 8 u + 4 + g (d1) of row r, in its half dsh / 16.
  uint4 qa, qb;
  uint32_t d0, d1;
  uint32_t dsh;  // 0 or 16
  struct Addr {
    uint32_t qa, qb, d, dsh;
    // The same lanes `rows` rows further on (rows may be negative). Rows
    // past the matrix are left past its planes, where the buffer loads
    // read zero, instead of being clamped to its last row.
    __device__ __forceinline__ void advance(int64_t rows, int64_t nb) {
      const int64_t blocks = rows * nb;
      const uint32_t dq = static_cast<uint32_t>(blocks * 16);
      qa += dq;
      qb += dq;
      const uint32_t od = d + (dsh >> 3) + static_cast<uint32_t>(blocks * 2);  // byte offset of the lane's d
      d = od & ~3u;
      dsh = (od & 2u) << 3;
    }
  };
  static __device__ __forceinline__ Addr addr(int64_t row0, int64_t n_rows, int64_t nb, int lane) {
    Addr a;
    const int h = lane >> 5, c = 4 * h + (lane & 3), rq = (lane & 31) >> 2;
    a.qa = static_cast<uint32_t>((min(row0 + rq, n_rows - 1) * nb + c) * 16);
    a.qb = static_cast<uint32_t>((min(row0 + 8 + rq, n_rows - 1) * nb + c) * 16);
    const uint32_t od = static_cast<uint32_t>((min(row0 + (lane & 15), n_rows - 1) * nb + (lane >> 4)) * 2);
    a.d = od & ~3u;
    a.dsh = (od & 2u) << 3;
    return a;
  }
  // Every load is issued and every value is a whole loaded dword (a load
  // under a branch, or a narrower load whose widening the compiler places
  // elsewhere, makes it wait for all of the ring's loads at once). Blocks
  // past nb (a k that is not a multiple of 256) read the next row's codes
  // and scales, or zero past the planes: every fp16 pattern decodes to a
  // finite scale, and the activations staged for k past the row are zero,
  // so those blocks add exact zeros.
  __device__ __forceinline__ void load(const Planes& P, const Addr& a, int64_t u, int64_t) {
    const uint32_t sq = static_cast<uint32_t>(u) * 128u, sd = static_cast<uint32_t>(u) * 16u;
    qa = bload16(P.a, a.qa, sq);
    qb = bload16(P.a, a.qb, sq);
    d0 = bload4(P.d, a.d, sd);
    d1 = bload4(P.d, a.d, sd + 8u);
    dsh = a.dsh;
  }
  // Once the unit's loads have arrived: qa <- step 0 of all 16 rows (rows
  // 0..7 in lanes 0..31, rows 8..15 in lanes 32..63), qb <- step 1. One
  // v_permlane32_swap a dword moves the upper half of qa and the lower half
  // of qb across, so each step's pieces then come from one register.
  __device__ __forceinline__ void arrange() {
    uint32_t a[4] = {qa.x, qa.y, qa.z, qa.w}, b[4] = {qb.x, qb.y, qb.z, qb.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const auto r = __builtin_amdgcn_permlane32_swap(a[j], b[j], false, false);
      a[j] = r[0];
      b[j] = r[1];
    }
    qa = make_uint4(a[0], a[1], a[2], a[3]);
    qb = make_uint4(b[0], b[1], b[2], b[3]);
  }
  // Piece of step h of the pair for MFMA lane (row lane % 16, group lane / 16)
  // (after arrange()).
  __device__ __forceinline__ void piece(MoePiece<SPIRAL_TYPE_Q4_0>& out, int h, int lane) const {
    const int r = lane & 15, g = lane >> 4;
    const int src = (32 * (r >> 3) + 4 * (r & 7) + g) << 2;
    const uint4 v = h ? qb : qa;
    const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
    uint32_t q[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) q[j] = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, static_cast<int>(vv[j])));
    out.q = make_uint4(q[0], q[1], q[2], q[3]);
    out.d = __builtin_amdgcn_ubfe(h ? d1 : d0, dsh, 16);
  }
};

// Routing shared by both forms: the expert's pairs as [begin, end) of lst.
// Fused (offsets == nullptr): a stable compaction of the pairs routed to e
// into s_list, in pair order, so every workgroup of the expert holds the same
// list (pass lanes split it between workgroups); expert 0's workgroups also
// clear the rows of pairs routed nowhere over columns [c0, c1).
template <bool F32_OUT>
__device__ __forceinline__ void moe_route(const int32_t* __restrict__ ids, int32_t n_pairs, int32_t n_expert,
                                          int64_t e, const int32_t* __restrict__ offsets,
                                          const int32_t* __restrict__ list, int32_t* s_list, int32_t& s_n,
                                          void* __restrict__ y, int64_t n_rows, int64_t c0, int64_t c1, int tid,
                                          int nthreads, int32_t& begin, int32_t& end, const int32_t*& lst) {
  if (offsets == nullptr) {
    __shared__ int32_t s_wave_hits[kMaxRouteWaves];
    const int wave = tid >> 6, lane = tid & 63, n_waves = nthreads >> 6;
    int32_t base = 0;
    for (int32_t p0 = 0; p0 < n_pairs; p0 += nthreads) {  // the same trip count in every thread
      const int32_t p = p0 + tid;
      const int32_t id = p < n_pairs ? ids[p] : -1;
      const uint64_t hits = __ballot(id == e);
      if (lane == 0) s_wave_hits[wave] = __popcll(hits);
      __syncthreads();
      int32_t before = 0, chunk = 0;
      for (int v = 0; v < n_waves; ++v) {
        before += v < wave ? s_wave_hits[v] : 0;
        chunk += s_wave_hits[v];
      }
      if (id == e) s_list[base + before + __popcll(hits & ((uint64_t(1) << lane) - 1))] = p;
      if (p < n_pairs && e == 0 && (id < 0 || id >= n_expert)) {
        for (int64_t c = c0; c < min(c1, n_rows); ++c) {
          if constexpr (F32_OUT)
            static_cast<float*>(y)[p * n_rows + c] = 0.0f;
          else
            static_cast<uint16_t*>(y)[p * n_rows + c] = 0;
        }
      }
      base += chunk;
      __syncthreads();  // s_wave_hits is rewritten by the next chunk
    }
    if (tid == 0) s_n = base;
    begin = 0;
    end = base;
    lst = s_list;
  } else {
    begin = offsets[e];
    end = offsets[e + 1];
    lst = list;
  }
}

// GLU: the fused form above (glu_op, swapped); the output then has n_rows / 2
// columns and the workgroups' row ranges are over those features.
//
// TB: MFMA row blocks per pass. A pass takes up to 16 TB of the expert's
// routed tokens, so every dequantized weight feeds TB MFMAs (prefill-sized
// batches read and dequantize each weight once per 16 TB tokens instead of
// once per 16). Pass lanes: workgroup (x, e, z) takes passes z, z + Z, ...
// of expert e (Z = gridDim.z), so the passes of a heavily routed expert run
// side by side.
template <int TYPE, bool F32_OUT, bool GLU, int TB, int WAVES>
__global__ void __launch_bounds__(64 * WAVES, (kStreamMinWaves<TYPE, TB, WAVES>)) moe_stream_kernel(
    const uint8_t* __restrict__ w, int64_t expert_stride, int64_t n_rows, int64_t k, const uint16_t* __restrict__ x,
    int64_t x_slots, int64_t top_k, const int32_t* __restrict__ ids, int32_t n_pairs, int32_t n_expert,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ list, void* __restrict__ y,
    int64_t rows_per_wg, int glu_op, int swapped, const uint8_t* __restrict__ w_up) {
  constexpr int kPass = kMoeTok * TB;  // tokens per pass
  constexpr uint32_t kEsize = F32_OUT ? 4 : 2, kOutSkip = 0x80000000u;
  extern __shared__ __align__(16) uint16_t As[];  // kPass rows of `pitch` bf16
  __shared__ int32_t s_pair[kPass];
  __shared__ int64_t s_xrow[kPass];
  __shared__ int32_t s_list[kFusedPairs];
  __shared__ int32_t s_n;
  constexpr int R = kStreamRing<TYPE>;
  const int64_t e = blockIdx.y;
  const int32_t lane_z = static_cast<int32_t>(blockIdx.z), n_lanes_z = static_cast<int32_t>(gridDim.z);
  const int tid = threadIdx.x, lane = tid & 63;
  const int64_t feat = GLU ? n_rows / 2 : n_rows;  // output columns
  const __amdgpu_buffer_rsrc_t Y = buffer_rsrc(y, static_cast<uint32_t>(static_cast<int64_t>(n_pairs) * feat * kEsize));
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * rows_per_wg;
  const int64_t r1 = min(r0 + rows_per_wg, feat);
  int32_t begin, end;
  const int32_t* lst;
  // Only pass lane 0 clears the rows of pairs routed nowhere (its columns).
  moe_route<F32_OUT>(ids, n_pairs, n_expert, e, offsets, list, s_list, s_n, y, feat, r0, lane_z == 0 ? r1 : r0, tid,
                     64 * WAVES, begin, end, lst);
  if (begin + lane_z * kPass >= end || r0 >= r1) return;

  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4;
  const int64_t nb = k / block_elems(TYPE);
  // 32-bit counters: the loop's tests stay scalar compares (64-bit ones are
  // VALU work on this GPU).
  const int steps = static_cast<int>((k + 127) / 128);
  const int pitch = steps * 128 + kAPad;
  // GLU split form (w_up set): gate rows in w, up rows in w_up, F rows each.
  const bool split = GLU && w_up != nullptr;
  const int64_t mat_rows = split ? feat : n_rows;  // rows of each expert matrix
  const Planes P = make_planes<TYPE>(w + e * expert_stride, mat_rows, nb);
  const Planes Pu = split ? make_planes<TYPE>(w_up + e * expert_stride, mat_rows, nb) : P;
  const int64_t up_row0 = split ? 0 : feat;  // first up row in its matrix
  // This wave's groups: ordinals j = 0 .. my_groups - 1, group wave + WAVES j.
  const int64_t groups = (r1 - r0 + 15) / 16;
  const int64_t my_groups = groups > wave ? (groups - wave + WAVES - 1) / WAVES : 0;
  const int units = (steps + Unit<TYPE>::kSteps - 1) / Unit<TYPE>::kSteps;
  const int gunits = GLU ? 2 * units : units;  // units per group: gate, then up
  const bool ragged = k % 128 != 0;
  const auto row_of = [&](int64_t j) { return r0 + 16 * (wave + WAVES * j) + (lane & 15); };

  for (int32_t t0 = begin + lane_z * kPass; t0 < end; t0 += n_lanes_z * kPass) {
    const int nt = min(kPass, end - t0);
    const int nblk = (nt + kMoeTok - 1) / kMoeTok;  // row blocks with routed tokens
    __syncthreads();
    if (tid < kPass) {
      const int32_t pr = tid < nt ? lst[t0 + tid] : -1;
      s_pair[tid] = pr;
      if (pr >= 0) {
        const int64_t t = pr / top_k, slot = pr % top_k;
        s_xrow[tid] = (t * x_slots + slot % x_slots) * k;
      }
    }
    // Weights do not depend on the tokens: fill the ring first. Load
    // pointer: unit (lj, lu) = (group ordinal, unit of the group). Every
    // ring load is issued, so the compiler can count the loads in flight
    // and wait for exactly the one it needs (a load under a branch makes it
    // wait for all of them); past the wave's last unit the ring re-reads it.
    using U = Unit<TYPE>;
    U ring[R];
    const int n_units = static_cast<int>(my_groups * gunits);
    int lj = 0, lu = 0, nl = 0;
    typename U::Addr la = U::addr(row_of(0) - (lane & 15), mat_rows, nb, lane);
    const auto issue = [&](int slot) {
      // Gate (or only) rows from P, up rows from Pu: a select of the buffer
      // descriptors, so the load itself is never under a branch.
      ring[slot].load(lu < units ? P : Pu, la, lu < units ? lu : lu - static_cast<int>(units), nb);
      if (++nl < n_units) {
        ++lu;
        // Q4_0 steps its offsets (a few 32-bit adds) where the other
        // formats recompute them from the row.
        if (GLU && lu == units) {  // up rows
          if constexpr (TYPE == SPIRAL_TYPE_Q4_0)
            la.advance(up_row0, nb);
          else
            la = U::addr(up_row0 + row_of(lj) - (lane & 15), mat_rows, nb, lane);
        }
        if (lu == gunits) {
          lu = 0;
          ++lj;
          if constexpr (TYPE == SPIRAL_TYPE_Q4_0)
            la.advance(16 * WAVES - (GLU ? up_row0 : 0), nb);
          else
            la = U::addr(row_of(lj) - (lane & 15), mat_rows, nb, lane);
        }
      }
    };
#pragma unroll
    for (int i = 0; i < R - 1; ++i) issue(i);
    __syncthreads();
    moe_stage<TYPE>(As, x, s_xrow, nt, k, 0, tid, static_cast<int>(steps * 128), pitch, 64 * WAVES);
    __syncthreads();

    // MFMA rows past nt read row nt - 1; their outputs are dropped.
    const uint16_t* arow[TB];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) arow[tb] = As + min(kMoeTok * tb + (lane & 15), nt - 1) * pitch + 8 * g;
    // Output row offsets of the lane's four pairs per row block (bytes; the
    // caller keeps y below 2 GiB): a pair that does not exist points past
    // the buffer (bit 31), where the buffer store drops its value.
    uint32_t yo[TB][4];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int32_t pr = s_pair[kMoeTok * tb + 4 * g + i];
        yo[tb][i] = pr >= 0 ? static_cast<uint32_t>(pr) * static_cast<uint32_t>(feat) * kEsize : kOutSkip;
      }
    f32x4_t acc[TB][4];
    f32x4_t gate[TB];  // GLU: the group's gate sums
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
#pragma unroll
      for (int s = 0; s < 4; ++s) acc[tb][s] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      gate[tb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
    int cj = 0, cu = 0;  // compute pointer
    const auto compute = [&](int slot) {
      const int ku = cu < units ? cu : cu - units;  // unit within the row
      ring[slot].arrange();
#pragma unroll
      for (int h = 0; h < U::kSteps; ++h) {
        const int st = ku * U::kSteps + h;
        if (U::kSteps == 1 || st < steps) {
          MoePiece<TYPE> pc;
          ring[slot].piece(pc, h, lane);
          if constexpr (TYPE != SPIRAL_TYPE_Q4_0 && TYPE != SPIRAL_TYPE_Q6_K) {
            // k tail: blocks past k read as zero
            if (ragged && st == steps - 1 && 32 * (4 * st + g) >= k) pc.zero();
          }
          pc.prep();
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const bf16x8_t b = __builtin_bit_cast(bf16x8_t, pc.dequant(s));
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
              if (TB == 1 || tb < nblk) {
                const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(arow[tb] + 8 * 16 * st + 8 * 4 * s);
                acc[tb][s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[tb][s], 0, 0, 0);
              }
            }
          }
        }
      }
      ++cu;
      if (GLU && cu == units) {
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
          gate[tb] = (acc[tb][0] + acc[tb][1]) + (acc[tb][2] + acc[tb][3]);
#pragma unroll
          for (int s = 0; s < 4; ++s) acc[tb][s] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
      } else if (cu == gunits) {
        // acc[tb]: lane l holds rows 16 tb + 4 (l / 16) + i (routed pairs) of
        // column l % 16. Every lane stores (no branch around the stores):
        // columns past the workgroup's range point past the buffer.
        const int64_t n = row_of(cj);
        const uint32_t n_off = static_cast<uint32_t>(n) * kEsize, n_skip = n < r1 ? 0u : kOutSkip;
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
          f32x4_t sum = (acc[tb][0] + acc[tb][1]) + (acc[tb][2] + acc[tb][3]);
          if constexpr (GLU) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              sum[i] = swapped ? glu_act(glu_op, sum[i]) * gate[tb][i] : glu_act(glu_op, gate[tb][i]) * sum[i];
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t off = (yo[tb][i] + n_off) | n_skip;
            if constexpr (F32_OUT)
              __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(sum[i]), Y, off, 0, 0);
            else
              __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, static_cast<__bf16>(sum[i])), Y,
                                                    off, 0, 0);
          }
#pragma unroll
          for (int s = 0; s < 4; ++s) acc[tb][s] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
        cu = 0;
        ++cj;
      }
    };
    // Whole rounds of R units (each issues the load R - 1 units ahead), then
    // the last units, which are already in the ring.
    int i0 = 0;
    for (; i0 + R <= n_units; i0 += R) {
#pragma unroll
      for (int d = 0; d < R; ++d) {
        issue((d + R - 1) % R);
        compute(d);
      }
    }
#pragma unroll
    for (int d = 0; d < R - 1; ++d) {
      if (i0 + d < n_units) compute(d);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // the ring's last (repeated) loads
}

// Dynamic LDS of the streaming form for k (0 when it does not fit).
// Dynamic LDS budget of the streaming form (the rest of the CU's 160 KiB
// holds its static arrays).
constexpr int64_t kStreamLdsMax = 150 * 1024;

// Dynamic LDS of the streaming form for k with tb row blocks per pass (0
// when it does not fit; tb = 1 fits every k <= kStreamMaxK).
int64_t stream_lds_bytes(int64_t k, int tb = 1) {
  if (k > kStreamMaxK) return 0;
  const int64_t bytes = int64_t(kMoeTok) * tb * (((k + 127) / 128) * 128 + kAPad) * 2;
  return bytes <= kStreamLdsMax ? bytes : 0;
}

// Row blocks per pass: enough for the average expert's routed tokens
// (prefill batches), as far as the activations of k fit in LDS.
int stream_tb(int64_t k, int64_t n_pairs, int64_t n_expert) {
  const int64_t avg = ceil_div(n_pairs, n_expert);
  if (avg > 2 * kMoeTok && stream_lds_bytes(k, 4) > 0) return 4;
  if (avg > kMoeTok && stream_lds_bytes(k, 2) > 0) return 2;
  return 1;
}

template <int TYPE, bool F32_OUT, bool GLU, int TB>
int launch_stream_tb(const void* w, int64_t expert_stride, int64_t n_expert, int64_t n_rows, int64_t k,
                     const uint16_t* x, int64_t x_slots, const int32_t* ids, int64_t n_pairs, int64_t top_k,
                     const int32_t* offsets, const int32_t* list, void* y, int glu_op, int swapped,
                     const void* w_up, hipStream_t s) {
  constexpr int kWaves = kStreamWaves<TYPE, GLU, TB>;
  const auto kern = moe_stream_kernel<TYPE, F32_OUT, GLU, TB, kWaves>;
  const int64_t lds = stream_lds_bytes(k, TB);
  const int64_t lds_max = TB == 1 ? stream_lds_bytes(kStreamMaxK) : kStreamLdsMax;
  const int rc = allow_dynamic_lds(reinterpret_cast<const void*>(kern), static_cast<int>(lds_max));
  if (rc != SPIRAL_OK) return rc;
  // Workgroups over contiguous ranges of whole 16-row groups of one expert
  // (GLU: of its output features), and pass lanes (grid z) for batches whose
  // average expert needs several passes. As many workgroups as the CUs hold
  // at once (at most two a CU), so each pass's activations are staged once
  // per CU; twice that with pass lanes, whose pass counts differ by one
  // between lanes of an expert, so that the dispatcher evens them out
  // (1024 tokens, top-8 over 128 experts, Q4_0 1536 x 2048: 203 us against
  // 246 us for one round and 218 us for four).
  const int64_t feat = GLU ? n_rows / 2 : n_rows;
  const int64_t lanes = std::min<int64_t>(8, std::max<int64_t>(1, ceil_div(n_pairs, n_expert * kMoeTok * TB)));
  const int64_t resident = static_cast<int64_t>(device_cu_count()) *
                           std::min(2, blocks_per_cu(reinterpret_cast<const void*>(kern), 64 * kWaves, lds));
  const int64_t rounds = lanes > 1 ? 2 : 1;
  const int64_t per_expert = std::max<int64_t>(1, ceil_div(rounds * resident, n_expert * lanes));
  const int64_t rows_per_wg = ceil_div(ceil_div(feat, per_expert), 16) * 16;
  const dim3 grid(static_cast<unsigned>(ceil_div(feat, rows_per_wg)), static_cast<unsigned>(n_expert),
                  static_cast<unsigned>(lanes));
  hipLaunchKernelGGL(kern, grid, dim3(64 * kWaves), static_cast<size_t>(lds), s, static_cast<const uint8_t*>(w),
                     expert_stride, n_rows, k, x, x_slots, top_k, ids, static_cast<int32_t>(n_pairs),
                     static_cast<int32_t>(n_expert), offsets, list, y, rows_per_wg, glu_op, swapped,
                     static_cast<const uint8_t*>(w_up));
  return launch_status();
}

template <int TYPE, bool F32_OUT, bool GLU>
int launch_stream(const void* w, int64_t expert_stride, int64_t n_expert, int64_t n_rows, int64_t k,
                  const uint16_t* x, int64_t x_slots, const int32_t* ids, int64_t n_pairs, int64_t top_k,
                  const int32_t* offsets, const int32_t* list, void* y, int glu_op, int swapped, const void* w_up,
                  hipStream_t s) {
  // The fused GLU form keeps TB <= 2 (four blocks of gate sums beside four
  // of accumulators exceed the registers of two waves a SIMD).
  const int tb = std::min(stream_tb(k, n_pairs, n_expert), GLU ? 2 : 4);
#define SPIRAL_STREAM_TB(TBV)                                                                                      \
  launch_stream_tb<TYPE, F32_OUT, GLU, TBV>(w, expert_stride, n_expert, n_rows, k, x, x_slots, ids, n_pairs, top_k, \
                                            offsets, list, y, glu_op, swapped, w_up, s)
  if constexpr (!GLU) {
    if (tb == 4) return SPIRAL_STREAM_TB(4);
  }
  if (tb == 2) return SPIRAL_STREAM_TB(2);
  return SPIRAL_STREAM_TB(1);
#undef SPIRAL_STREAM_TB
}

// ---- dense small-batch form (ggml MUL_MAT with 2 .. 16 rows of x) --------
//
// The streaming form without routing: the m <= kMoeTok rows of x are the
// MFMA A rows, and every weight byte is read once. A dense matrix has far
// fewer 16-row groups than the chip has waves (256 for 4096 rows), so the 8
// waves of a workgroup work on a "block" of 8 / parts groups, `parts` waves
// per group, each over its own slice of k; the slices' partial sums meet in
// LDS at the end of the block (in slice order, so results do not depend on
// timing). Workgroups are persistent: workgroup b takes blocks b, b + grid,
// ..., stages x once and streams its blocks end to end through each wave's
// register ring, whose loads run ahead across block ends.
//
// Windows: when m rows of x over the whole k do not fit the LDS budget, k is
// cut into n_win windows of whole units (balanced, each holding at least
// `parts` units), staged one after the other within every block; every wave
// owns a slice of every window, so all waves meet the same barriers. Weight
// loads do not depend on x, so the ring keeps running across window ends.
constexpr int kSkinnyThreads = 512;
constexpr int kSkinnyWaves = kSkinnyThreads / 64;
constexpr int64_t kSkinnyLds = 152 * 1024;               // activation window + partial sums
constexpr int kSkinnyRed = 2 * kSkinnyWaves * 4 * 64 * 4;  // partial sums, two blocks' worth

struct SkinnyShape {
  int parts, n_win;
  int64_t groups, units, win_units, lds;
};

// WINDOWS: n_win > 1 (restaging inside the loop). Without it the loop body
// issues no memory instruction under a branch: the output stores are buffer
// stores that every lane executes (lanes with nothing to store point past the
// buffer, and the hardware drops them), so the compiler can count the ring's
// loads in flight and wait for exactly the one it needs.
template <int TYPE, bool F32_OUT, bool WINDOWS>
__global__ void __launch_bounds__(kSkinnyThreads) skinny_kernel(const uint8_t* __restrict__ w, int64_t n_rows,
                                                                int64_t k, const uint16_t* __restrict__ x,
                                                                int64_t ldx, int m, void* __restrict__ y,
                                                                int64_t ldy, int parts, int n_win, int pitch) {
  extern __shared__ __align__(16) uint16_t As[];  // m rows of `pitch` bf16, then the partial sums
  __shared__ int64_t s_xrow[kMoeTok];
  using U = Unit<TYPE>;
  constexpr int R = kStreamRing<TYPE>;
  constexpr uint32_t kEsize = F32_OUT ? 4 : 2;
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int per_block = kSkinnyWaves / parts;
  const int gslot = wave / parts, part = wave - gslot * parts;
  const int64_t groups = (n_rows + 15) / 16;
  const int64_t n_blocks = (groups + per_block - 1) / per_block;
  // blocks blockIdx.x + gridDim.x i, i < my_blocks (the grid is at most n_blocks)
  const int my_blocks = static_cast<int>((n_blocks - 1 - blockIdx.x) / gridDim.x + 1);
  const auto row0_of = [&](int i) {
    return ((static_cast<int64_t>(blockIdx.x) + static_cast<int64_t>(gridDim.x) * i) * per_block + gslot) * 16;
  };
  const int64_t nb = k / block_elems(TYPE);
  const int steps = static_cast<int>((k + 127) / 128);
  const int units = (steps + U::kSteps - 1) / U::kSteps;
  const Planes P = make_planes<TYPE>(w, n_rows, nb);
  // y as a buffer of (m - 1) ldy + n_rows elements (below 2^31 bytes)
  const __amdgpu_buffer_rsrc_t Y = buffer_rsrc(y, static_cast<uint32_t>(((m - 1) * ldy + n_rows) * kEsize));
  float* red = reinterpret_cast<float*>(As + m * pitch);  // [2][8 waves][4][64]
  if (tid < kMoeTok) s_xrow[tid] = static_cast<int64_t>(min(tid, m - 1)) * ldx;

  // Window v holds units [wb(v), wb(v + 1)); this wave owns slice(v, part) .. slice(v, part + 1).
  const auto wb = [&](int v) {
    return WINDOWS ? static_cast<int>(static_cast<int64_t>(units) * v / n_win) : v * units;
  };
  const auto slice = [&](int v, int p) { return wb(v) + (wb(v + 1) - wb(v)) * p / parts; };
  int per_blk_units = 0;
  for (int v = 0; v < (WINDOWS ? n_win : 1); ++v) per_blk_units += slice(v, part + 1) - slice(v, part);
  const int n_units = my_blocks * per_blk_units;

  // Load pointer: block lb, window lv, unit lu, end of this wave's slice le.
  U ring[R];
  typename U::Addr la = U::addr(row0_of(0), n_rows, nb, lane);
  int lb = 0, lv = 0, lu = slice(0, part), le = slice(0, part + 1), nl = 0;
  const auto issue = [&](int s) {
    ring[s].load(P, la, lu, nb);
    if (++nl < n_units && ++lu == le) {  // past the last unit the ring re-reads it
      if (!WINDOWS || ++lv == n_win) {
        lv = 0;
        ++lb;
        if constexpr (TYPE == SPIRAL_TYPE_Q4_0)
          la.advance(static_cast<int64_t>(gridDim.x) * per_block * 16, nb);
        else
          la = U::addr(row0_of(lb), n_rows, nb, lane);
      }
      lu = slice(lv, part);
      le = slice(lv, part + 1);
    }
  };
  const auto stage = [&](int v) {
    const int64_t c0 = static_cast<int64_t>(wb(v)) * U::kSteps * 128;
    const int width = (wb(v + 1) - wb(v)) * U::kSteps * 128;
    moe_stage<TYPE>(As, x, s_xrow, m, k, c0, tid, width, pitch, kSkinnyThreads);
  };
  // x first: its loads complete in order ahead of the ring's.
  __syncthreads();
  stage(0);
#pragma unroll
  for (int i = 0; i < R - 1; ++i) issue(i);
  __syncthreads();

  // MFMA rows past m read row m - 1; their outputs are dropped.
  const uint16_t* arow = As + min(lane & 15, m - 1) * pitch + 8 * g;
  f32x4_t acc[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) acc[s] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  int cb = 0, cv = 0, cu = slice(0, part), ce = slice(0, part + 1);  // compute pointer
  int64_t st0 = 0;                                                   // first k step of window cv
  const bool ragged = k % 128 != 0;
  const auto finish_block = [&]() {
    // acc: lane l holds x rows 4 (l / 16) + i of weight row row0 + l % 16.
    f32x4_t sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    float* rb = red + (cb & 1) * (kSkinnyWaves * 4 * 64);
    // With k slices (parts > 1), slice 0's wave sums and stores x rows
    // 4 g + 0, 1 of the group and slice 1's rows 4 g + 2, 3; the other
    // slices' waves repeat one of the two sums and store nothing. Each sum
    // adds the slices in slice order, so results do not depend on timing.
    const int i0 = 2 * (part & 1);
    if (parts > 1) {
#pragma unroll
      for (int i = 0; i < 4; ++i) rb[(wave * 4 + i) * 64 + lane] = sum[i];
      // every wave is done with this block's partial sums (and with x)
      __syncthreads();
      const float* rg = rb + (gslot * parts * 4 + i0) * 64 + lane;
      float s0 = rg[0], s1 = rg[64];
      for (int p = 1; p < parts; ++p) {
        s0 += rg[p * 4 * 64];
        s1 += rg[p * 4 * 64 + 64];
      }
      sum = i0 ? f32x4_t{sum[0], sum[1], s0, s1} : f32x4_t{s0, s1, sum[2], sum[3]};
    } else if (WINDOWS && cb + 1 < my_blocks) {
      __syncthreads();  // every wave is done with x
    }
    // Lanes with nothing to store set bit 31 of the offset (past the buffer);
    // bit arithmetic, not a select, so no branch forms around the stores.
    const int64_t n = row0_of(cb) + (lane & 15);
    const uint32_t skip = static_cast<uint32_t>(n >= n_rows);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 4 * g + i;
      const uint32_t mine = static_cast<uint32_t>(parts == 1) | (static_cast<uint32_t>(part < 2) &
                                                                    static_cast<uint32_t>((i >> 1) == part));
      const uint32_t bad = (skip | (mine ^ 1u) | static_cast<uint32_t>(t >= m)) << 31;
      const uint32_t off = (static_cast<uint32_t>(min(t, m - 1) * ldy + min(n, n_rows - 1)) * kEsize) | bad;
      if constexpr (F32_OUT)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(sum[i]), Y, off, 0, 0);
      else
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, static_cast<__bf16>(sum[i])), Y, off, 0,
                                              0);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) acc[s] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    if (WINDOWS && cb + 1 < my_blocks) {
      stage(0);
      __syncthreads();
    }
    ++cb;
  };
  const auto compute = [&](int slot) {
    ring[slot].arrange();
#pragma unroll
    for (int h = 0; h < U::kSteps; ++h) {
      const int st = cu * U::kSteps + h;
      if (U::kSteps == 1 || st < steps) {
        MoePiece<TYPE> pc;
        ring[slot].piece(pc, h, lane);
        if constexpr (TYPE != SPIRAL_TYPE_Q4_0 && TYPE != SPIRAL_TYPE_Q6_K) {
          if (ragged && st == steps - 1 && 32 * (4 * st + g) >= k) pc.zero();
        }
        pc.prep();
        const uint16_t* ak = arow + 8 * 16 * (st - st0);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const bf16x8_t b = __builtin_bit_cast(bf16x8_t, pc.dequant(s));
          const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(ak + 8 * 4 * s);
          acc[s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[s], 0, 0, 0);
        }
      }
    }
    if (++cu == ce) {
      if (WINDOWS && cv + 1 < n_win) {
        // next window: every wave is done with this one before it is replaced
        ++cv;
        __syncthreads();
        stage(cv);
        __syncthreads();
      } else {
        finish_block();
        cv = 0;
      }
      cu = slice(cv, part);
      ce = slice(cv, part + 1);
      st0 = static_cast<int64_t>(wb(cv)) * U::kSteps;
    }
  };
  int i0 = 0;
  for (; i0 + R <= n_units; i0 += R) {
#pragma unroll
    for (int d = 0; d < R; ++d) {
      issue((d + R - 1) % R);
      compute(d);
    }
  }
#pragma unroll
  for (int d = 0; d < R - 1; ++d) {
    if (i0 + d < n_units) compute(d);
  }
  __builtin_amdgcn_s_waitcnt(0);  // the ring's last (repeated) loads
}

// Slices of k per group and windows of k for m rows of x (parts = 0: the
// shape does not fit this form).
SkinnyShape skinny_shape(int type, int64_t n_rows, int64_t k, int64_t m) {
  SkinnyShape sh{};
  const int64_t ksteps = type == SPIRAL_TYPE_Q4_0 ? 2 : 1;
  sh.groups = ceil_div(n_rows, 16);
  sh.units = ceil_div(ceil_div(k, 128), ksteps);
  // Widest window (in units) whose activations fit next to the partial sums.
  const int64_t fit = ((kSkinnyLds - kSkinnyRed) / (2 * m) - kAPad) / (128 * ksteps);
  if (fit < 1) return sh;
  sh.n_win = static_cast<int>(ceil_div(sh.units, fit));
  sh.win_units = ceil_div(sh.units, sh.n_win);
  // The most slices the windows allow (up to one wave per slice); the
  // launch picks among the powers of two up to it (skinny_parts).
  const int64_t min_win = sh.units / sh.n_win;
  int parts = 1;
  while (parts < kSkinnyWaves && 2 * parts <= min_win) parts *= 2;
  sh.parts = parts;
  sh.lds = 2 * m * (128 * ksteps * sh.win_units + kAPad) + kSkinnyRed;
  return sh;
}

// k slices per 16-row group for `resident` workgroups at once. sh.parts is
// the most the windows allow; a launch takes the count that gives the
// busiest wave the fewest units, and among those the fewest block ends (a
// block end is an LDS exchange of partial sums behind a barrier, about
// 0.6 us at m = 4 on 14336 x 4096 Q4_0: 8 slices (four blocks a workgroup)
// took 15.8 us, 4 slices 14.3 and 2 slices (one block) 13.9, every choice
// giving the busiest wave 8 units).
int skinny_parts(const SkinnyShape& sh, int64_t resident) {
  int best = sh.parts;
  int64_t best_units = INT64_MAX, best_ends = INT64_MAX;
  for (int p = 1; p <= sh.parts; p *= 2) {
    const int64_t n_blocks = ceil_div(sh.groups, kSkinnyWaves / p);
    const int64_t wgs = std::min(n_blocks, std::max<int64_t>(1, resident));
    const int64_t ends = ceil_div(n_blocks, wgs);             // blocks of the busiest workgroup
    const int64_t units = ends * sh.n_win * ceil_div(sh.win_units, p);  // its waves' units, at most
    if (units < best_units || (units == best_units && ends < best_ends)) {
      best = p;
      best_units = units;
      best_ends = ends;
    }
  }
  return best;
}

template <int TYPE, bool F32_OUT, bool WINDOWS>
int launch_skinny(const void* w, int64_t n_rows, int64_t k, const uint16_t* x, int64_t ldx, int64_t m, void* y,
                  int64_t ldy, const SkinnyShape& sh, hipStream_t s) {
  const auto kern = skinny_kernel<TYPE, F32_OUT, WINDOWS>;
  const int rc = allow_dynamic_lds(reinterpret_cast<const void*>(kern), static_cast<int>(kSkinnyLds));
  if (rc != SPIRAL_OK) return rc;
  const int64_t resident =
      static_cast<int64_t>(device_cu_count()) * blocks_per_cu(reinterpret_cast<const void*>(kern), kSkinnyThreads, sh.lds);
  const int parts = skinny_parts(sh, resident);
  const int64_t n_blocks = ceil_div(sh.groups, kSkinnyWaves / parts);
  const int pitch = static_cast<int>(128 * Unit<TYPE>::kSteps * sh.win_units + kAPad);
  const dim3 grid(static_cast<unsigned>(std::min(n_blocks, resident)));
  hipLaunchKernelGGL(kern, grid, dim3(kSkinnyThreads), static_cast<size_t>(sh.lds), s,
                     static_cast<const uint8_t*>(w), n_rows, k, x, ldx, static_cast<int>(m), y, ldy, parts,
                     sh.n_win, pitch);
  return launch_status();
}

}  // namespace

// Whether the dense small-batch form takes this product.
bool skinny_fits(int type, int64_t n_rows, int64_t k, int64_t m) {
  if (m < 2 || m > kMoeTok) return false;
  // weight planes are addressed with 32-bit offsets, past-the-end reads at 2^31
  const int64_t wbytes = spiral_tensor_bytes(type, n_rows, k);
  if (wbytes == 0 || wbytes >= (int64_t(1) << 31)) return false;
  return skinny_shape(type, n_rows, k, m).parts > 0;
}

// Arguments validated by the caller; skinny_fits() holds.
int skinny(int type, const void* w, int64_t n_rows, int64_t k, const uint16_t* x, int64_t ldx, int64_t m, void* y,
           int y_type, int64_t ldy, hipStream_t s) {
  const SkinnyShape sh = skinny_shape(type, n_rows, k, m);
  const bool f32 = y_type == SPIRAL_TYPE_F32;
  // y is written through a buffer resource with 32-bit offsets
  if (((m - 1) * ldy + n_rows) * (f32 ? 4 : 2) >= (int64_t(1) << 31)) return SPIRAL_ERR_SHAPE;
#define SPIRAL_SKINNY(T)                                                                     \
  do {                                                                                        \
    if (sh.n_win > 1)                                                                         \
      return f32 ? launch_skinny<T, true, true>(w, n_rows, k, x, ldx, m, y, ldy, sh, s)      \
                 : launch_skinny<T, false, true>(w, n_rows, k, x, ldx, m, y, ldy, sh, s);    \
    return f32 ? launch_skinny<T, true, false>(w, n_rows, k, x, ldx, m, y, ldy, sh, s)       \
               : launch_skinny<T, false, false>(w, n_rows, k, x, ldx, m, y, ldy, sh, s);     \
  } while (0)
  if (type == SPIRAL_TYPE_Q4_0) SPIRAL_SKINNY(SPIRAL_TYPE_Q4_0);
  if (type == SPIRAL_TYPE_Q8_0) SPIRAL_SKINNY(SPIRAL_TYPE_Q8_0);
  if (type == SPIRAL_TYPE_Q4_K) SPIRAL_SKINNY(SPIRAL_TYPE_Q4_K);
  if (type == SPIRAL_TYPE_Q5_K) SPIRAL_SKINNY(SPIRAL_TYPE_Q5_K);
  if (type == SPIRAL_TYPE_IQ4_NL) SPIRAL_SKINNY(SPIRAL_TYPE_IQ4_NL);
  if (type == SPIRAL_TYPE_IQ4_XS) SPIRAL_SKINNY(SPIRAL_TYPE_IQ4_XS);
  SPIRAL_SKINNY(SPIRAL_TYPE_Q6_K);
#undef SPIRAL_SKINNY
}

int64_t moe_workspace_bytes(int64_t n_expert, int64_t n_pairs) { return 4 * (n_expert + 1 + n_pairs); }

// Whether the fused GLU form (streaming kernel only) takes rows of k elements.
bool moe_glu_fits_k(int64_t k) { return stream_lds_bytes(k) > 0; }

// ---- library-owned routing scratch (spiral_mul_mat_id_noalloc) -------------
//
// One array per GPU, in the code object's device memory, for callers that
// cannot allocate: the routing lists of a MUL_MAT_ID (offsets and list, see
// route_kernel) go here instead of a caller workspace. route_kernel writes
// every entry it later reads, so nothing needs clearing between calls. In
// host code `scratch` only names the symbol; its device address comes from
// hipGetSymbolAddress, once per device (each GPU has its own copy).
static __device__ __align__(256) uint8_t scratch[SPIRAL_MUL_MAT_ID_STATIC_BYTES];

// Device address of the current device's scratch (looked up once per device
// under a lock), or nullptr with rc set.
void* moe_static_scratch(int& rc) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    rc = SPIRAL_ERR_HIP;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      rc = SPIRAL_ERR_HIP;
      return nullptr;
    }
    addr[dev] = p;
  }
  rc = SPIRAL_OK;
  return addr[dev];
}

// Arguments validated by the caller. glu_op < 0: plain MUL_MAT_ID; otherwise
// the fused GLU form (n_rows = 2F even), which only the streaming form
// implements (k <= kStreamMaxK and y below 2 GiB, else SPIRAL_ERR_SHAPE):
// gate rows [0, F) and up rows [F, 2F) of each expert matrix, or, with w_up
// set (ggml's split form), the F rows of w and of w_up, both at
// expert_stride.
int moe(int type, const void* w, int64_t expert_stride, int64_t n_expert, int64_t n_rows, int64_t k,
        const uint16_t* x, int64_t x_slots, const int32_t* ids, int64_t n_tokens, int64_t top_k, void* y,
        int y_type, int glu_op, int swapped, void* workspace, hipStream_t s, const void* w_up) {
  const int64_t n_pairs = n_tokens * top_k;
  const int f32 = y_type == SPIRAL_TYPE_F32;
  const bool glu = glu_op >= 0;
  // Weight planes of one expert are addressed with 32-bit offsets.
  const int64_t wbytes = spiral_tensor_bytes(type, n_rows, k);
  if (wbytes == 0 || wbytes >= (int64_t(1) << 31)) return SPIRAL_ERR_SHAPE;
  // The streaming form writes y through a buffer resource (32-bit offsets).
  const int64_t y_bytes = n_pairs * (glu ? n_rows / 2 : n_rows) * (f32 ? 4 : 2);
  const bool stream_ok = stream_lds_bytes(k) > 0 && y_bytes < (int64_t(1) << 31);
  if (glu && !stream_ok) return SPIRAL_ERR_SHAPE;
  int32_t* offsets = nullptr;
  int32_t* list = nullptr;
  if (n_pairs > kFusedPairs) {
    offsets = static_cast<int32_t*>(workspace);
    list = offsets + n_expert + 1;
    hipLaunchKernelGGL(route_kernel, dim3(1), dim3(kRouteThreads), 0, s, ids, static_cast<int32_t>(n_pairs),
                       static_cast<int32_t>(n_expert), offsets, list, y, glu ? n_rows / 2 : n_rows, f32);
    if (hipGetLastError() != hipSuccess) return SPIRAL_ERR_HIP;
  }
  if (stream_ok) {
#define SPIRAL_MOE_STREAM_AS(T, F, G) \
  launch_stream<T, F, G>(w, expert_stride, n_expert, n_rows, k, x, x_slots, ids, n_pairs, top_k, offsets, list, y, \
                         glu_op, swapped, w_up, s)
#define SPIRAL_MOE_STREAM(T)                                                                                 \
  do {                                                                                                       \
    if (glu) return f32 ? SPIRAL_MOE_STREAM_AS(T, true, true) : SPIRAL_MOE_STREAM_AS(T, false, true);        \
    return f32 ? SPIRAL_MOE_STREAM_AS(T, true, false) : SPIRAL_MOE_STREAM_AS(T, false, false);               \
  } while (0)
    if (type == SPIRAL_TYPE_Q4_0) SPIRAL_MOE_STREAM(SPIRAL_TYPE_Q4_0);
    if (type == SPIRAL_TYPE_Q8_0) SPIRAL_MOE_STREAM(SPIRAL_TYPE_Q8_0);
    if (type == SPIRAL_TYPE_Q4_K) SPIRAL_MOE_STREAM(SPIRAL_TYPE_Q4_K);
    if (type == SPIRAL_TYPE_Q5_K) SPIRAL_MOE_STREAM(SPIRAL_TYPE_Q5_K);
    if (type == SPIRAL_TYPE_IQ4_NL) SPIRAL_MOE_STREAM(SPIRAL_TYPE_IQ4_NL);
    if (type == SPIRAL_TYPE_IQ4_XS) SPIRAL_MOE_STREAM(SPIRAL_TYPE_IQ4_XS);
    SPIRAL_MOE_STREAM(SPIRAL_TYPE_Q6_K);
#undef SPIRAL_MOE_STREAM
#undef SPIRAL_MOE_STREAM_AS
  }
  const dim3 grid(static_cast<unsigned>(ceil_div(n_rows, kMoeBN)), static_cast<unsigned>(n_expert));
  const uint8_t* W = static_cast<const uint8_t*>(w);
#define SPIRAL_MOE(T)                                                                                    \
  do {                                                                                                   \
    if (f32)                                                                                             \
      hipLaunchKernelGGL((moe_kernel<T, true>), grid, dim3(256), 0, s, W, expert_stride, n_rows, k, x,   \
                         x_slots, top_k, ids, static_cast<int32_t>(n_pairs), static_cast<int32_t>(n_expert), \
                         offsets, list, y);                                                              \
    else                                                                                                 \
      hipLaunchKernelGGL((moe_kernel<T, false>), grid, dim3(256), 0, s, W, expert_stride, n_rows, k, x,  \
                         x_slots, top_k, ids, static_cast<int32_t>(n_pairs), static_cast<int32_t>(n_expert), \
                         offsets, list, y);                                                              \
  } while (0)
  if (type == SPIRAL_TYPE_Q4_0) SPIRAL_MOE(SPIRAL_TYPE_Q4_0);
  else if (type == SPIRAL_TYPE_Q8_0) SPIRAL_MOE(SPIRAL_TYPE_Q8_0);
  else if (type == SPIRAL_TYPE_Q4_K) SPIRAL_MOE(SPIRAL_TYPE_Q4_K);
  else if (type == SPIRAL_TYPE_Q5_K) SPIRAL_MOE(SPIRAL_TYPE_Q5_K);
  else if (type == SPIRAL_TYPE_IQ4_NL) SPIRAL_MOE(SPIRAL_TYPE_IQ4_NL);
  else if (type == SPIRAL_TYPE_IQ4_XS) SPIRAL_MOE(SPIRAL_TYPE_IQ4_XS);
  else SPIRAL_MOE(SPIRAL_TYPE_Q6_K);
#undef SPIRAL_MOE
  return launch_status();
}

// Standalone GLU over `rows` rows of 2n floats; arguments validated by the
// caller.
int glu(int op, int swapped, const float* x, int64_t ldx, int64_t n, int64_t rows, float* y, int64_t ldy,
        hipStream_t s, float alpha, float limit) {
  const int64_t total = n * rows;
  if (total == 0) return SPIRAL_OK;
  const int64_t blocks = std::min<int64_t>(ceil_div(total, 256), 8 * static_cast<int64_t>(device_cu_count()));
  hipLaunchKernelGGL(glu_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, x, ldx, y, ldy, n, rows, op,
                     swapped, alpha, limit);
  return launch_status();
}

// Split form: gate rows at xg (stride ldg), up rows at xu (stride ldu).
int glu_split(int op, int swapped, const float* xg, int64_t ldg, const float* xu, int64_t ldu, int64_t n,
              int64_t rows, float* y, int64_t ldy, hipStream_t s, float alpha, float limit) {
  const int64_t total = n * rows;
  if (total == 0) return SPIRAL_OK;
  const int64_t blocks = std::min<int64_t>(ceil_div(total, 256), 8 * static_cast<int64_t>(device_cu_count()));
  hipLaunchKernelGGL(glu_split_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, xg, ldg, xu, ldu, y, ldy,
                     n, rows, op, swapped, alpha, limit);
  return launch_status();
}

}  // namespace spiral
