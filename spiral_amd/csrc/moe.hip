// Grouped dequant-GEMM for mixture-of-experts (ggml MUL_MAT_ID with
// quantized, expert-stacked weights).
//
// Two launches on the caller's stream:
//  1. route_kernel (one workgroup): a counting sort of the (token, slot)
//     pairs by expert id into per-expert lists in the caller's workspace;
//     pairs with an out-of-range id get a zero output row.
//  2. moe_kernel: workgroup (n-tile of 64 rows, expert) streams those weight
//     rows and multiplies them against the tokens routed to the expert, 16
//     tokens (one MFMA row block) per pass. At decode batch sizes (a few
//     tokens per expert) that is one pass, so each expert's weights are read
//     from HBM once per call, which is what bounds this op.
//
// moe_kernel layout (gfx950, v_mfma_f32_16x16x32_bf16):
//  - Wave w owns weight rows n0 + 16 w .. + 15 (the MFMA B columns). Lane l
//    serves row l % 16 and k-group g = l / 16. For every 128-wide k step it
//    loads one piece per lane (Q4_0 / Q8_0: block 4 kb + g; Q6_K: 32-element
//    group g of the half super-block) straight from HBM and dequantizes it
//    into the B operands of the step's four MFMAs, so weights never touch
//    LDS. Pieces are requested kMoeRing - 1 steps ahead (register ring).
//  - An MFMA sums over its 32 k in any order as long as A and B agree; MFMA
//    s of a step takes, from lane group g, the 8 elements of piece g that
//    are cheapest to unpack (see MoePiece). The routed tokens' activations
//    are staged per 1024-wide k chunk in LDS in exactly that order (only the
//    pass's real token rows; MFMA rows past them read a copy and their
//    outputs are dropped).
// Products use exactly dequantized bf16 weights and fp32 accumulation, as in
// the dense GEMM.
#include "common.h"
#include "dequant_impl.h"

namespace spiral {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int kRouteThreads = 1024;
constexpr int kRouteChunk = 4096;  // experts counted per LDS pass
constexpr int kMoeBN = 64;  // weight rows per workgroup (16 per wave)

// Workspace: offsets[n_expert + 1] then list[n_pairs] (int32).
//
// One workgroup: per chunk of kRouteChunk experts, count the pairs of each
// expert with LDS atomics, turn the counts into list offsets with a block
// scan, then scatter each pair's index into its expert's list. The order
// inside a list is arbitrary; each output row is computed on its own, so it
// does not change any result. Pairs with an id outside [0, n_expert) get a
// zero output row.
__global__ void __launch_bounds__(kRouteThreads) route_kernel(const int32_t* __restrict__ ids, int32_t n_pairs,
                                                              int32_t n_expert, int32_t* __restrict__ offsets,
                                                              int32_t* __restrict__ list, void* __restrict__ y,
                                                              int64_t n_rows, int y_f32) {
  __shared__ int32_t s_cnt[kRouteChunk];
  __shared__ int32_t s_wave[kRouteThreads / 64];
  __shared__ int32_t s_bad[kRouteThreads];
  __shared__ int32_t s_nbad;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  constexpr int kPer = kRouteChunk / kRouteThreads;
  int32_t base = 0;
  for (int32_t e0 = 0; e0 < n_expert; e0 += kRouteChunk) {
    const int32_t ne = min(kRouteChunk, n_expert - e0);
    for (int i = tid; i < kRouteChunk; i += kRouteThreads) s_cnt[i] = 0;
    __syncthreads();
    for (int32_t p = tid; p < n_pairs; p += kRouteThreads) {
      const int32_t e = ids[p] - e0;
      if (e >= 0 && e < ne) atomicAdd(&s_cnt[e], 1);
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
    for (int32_t p = tid; p < n_pairs; p += kRouteThreads) {
      const int32_t e = ids[p] - e0;
      if (e >= 0 && e < ne) list[atomicAdd(&s_cnt[e], 1)] = p;
    }
    base += total;
    __syncthreads();
  }
  if (tid == 0) offsets[n_expert] = base;
  // Pairs routed nowhere produce a zero row: collect them kRouteThreads at a
  // time, then clear their rows with the whole workgroup.
  for (int32_t p0 = 0; p0 < n_pairs; p0 += kRouteThreads) {
    if (tid == 0) s_nbad = 0;
    __syncthreads();
    const int32_t p = p0 + tid;
    if (p < n_pairs) {
      const int32_t e = ids[p];
      if (e < 0 || e >= n_expert) s_bad[atomicAdd(&s_nbad, 1)] = p;
    }
    __syncthreads();
    const int32_t nbad = s_nbad;
    for (int32_t b = 0; b < nbad; ++b) {
      const int64_t row = s_bad[b];
      for (int64_t col = tid; col < n_rows; col += kRouteThreads) {
        if (y_f32)
          static_cast<float*>(y)[row * n_rows + col] = 0.0f;
        else
          static_cast<uint16_t*>(y)[row * n_rows + col] = 0;
      }
    }
    __syncthreads();
  }
}

// One 128-wide k step of one weight row for lane group g (see the header):
// loaded once, then dequantized 8 elements at a time for MFMA s = 0..3.
// local(g, s, e) is the k offset inside the step of element e < 8 of MFMA s.
template <int TYPE>
struct MoePiece;

// Q4_0: piece = block 4 kb + g. MFMA s takes qs dword s: its low nibbles
// (elements 4s .. 4s + 3) then its high nibbles (16 + 4s .. 16 + 4s + 3).
template <>
struct MoePiece<SPIRAL_TYPE_Q4_0> {
  uint4 q;
  uint32_t d;
  static __device__ __forceinline__ int local(int g, int s, int e) { return 32 * g + (e < 4 ? 4 * s + e : 12 + 4 * s + e); }
  // blk = block index of the lane's piece within the row's planar planes
  __device__ __forceinline__ void load(const uint8_t* we, int64_t tot, int64_t blk) {
    q = *reinterpret_cast<const uint4*>(we + blk * 16);
    d = *reinterpret_cast<const uint16_t*>(we + tot * 16 + blk * 2);
  }
  __device__ __forceinline__ void zero() { q = make_uint4(0u, 0u, 0u, 0u); d = 0u; }
  __device__ __forceinline__ uint4 dequant(int s) const {
    const uint32_t w = s == 0 ? q.x : s == 1 ? q.y : s == 2 ? q.z : q.w;
    const float df = fp16_scale(d), off = -1032.0f * df;
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t c = i ? hi : lo;
      const f16x2_t a = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, c, 0x04010400u));
      const f16x2_t b = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, c, 0x04030402u));
      o[2 * i] = pack_bf16x2(__builtin_fmaf(static_cast<float>(a.x), df, off), __builtin_fmaf(static_cast<float>(a.y), df, off));
      o[2 * i + 1] = pack_bf16x2(__builtin_fmaf(static_cast<float>(b.x), df, off), __builtin_fmaf(static_cast<float>(b.y), df, off));
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
  }
};

// Q8_0: piece = block 4 kb + g; MFMA s takes qs bytes 8s .. 8s + 7.
template <>
struct MoePiece<SPIRAL_TYPE_Q8_0> {
  uint4 q0, q1;
  uint32_t d;
  static __device__ __forceinline__ int local(int g, int s, int e) { return 32 * g + 8 * s + e; }
  __device__ __forceinline__ void load(const uint8_t* we, int64_t tot, int64_t blk) {
    q0 = *reinterpret_cast<const uint4*>(we + blk * 32);
    q1 = *reinterpret_cast<const uint4*>(we + blk * 32 + 16);
    d = *reinterpret_cast<const uint16_t*>(we + tot * 32 + blk * 2);
  }
  __device__ __forceinline__ void zero() { q0 = q1 = make_uint4(0u, 0u, 0u, 0u); d = 0u; }
  __device__ __forceinline__ uint4 dequant(int s) const {
    const uint32_t w0 = (s == 0 ? q0.x : s == 1 ? q0.z : s == 2 ? q1.x : q1.z) ^ 0x80808080u;
    const uint32_t w1 = (s == 0 ? q0.y : s == 1 ? q0.w : s == 2 ? q1.y : q1.w) ^ 0x80808080u;
    const float df = fp16_scale(d), off = -1152.0f * df;
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t c = i ? w1 : w0;
      const f16x2_t a = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, c, 0x04010400u));
      const f16x2_t b = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, c, 0x04030402u));
      o[2 * i] = pack_bf16x2(__builtin_fmaf(static_cast<float>(a.x), df, off), __builtin_fmaf(static_cast<float>(a.y), df, off));
      o[2 * i + 1] = pack_bf16x2(__builtin_fmaf(static_cast<float>(b.x), df, off), __builtin_fmaf(static_cast<float>(b.y), df, off));
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
  }
};

// Q6_K: a 128-wide step is half h of super-block sb; piece g = elements
// 128 h + 32 g + l, l < 32 (ql[64 h + 32 (g & 1) + l] nibble g / 2, qh[32 h
// + l] bits 2g, sub-scale sc[8 h + l / 16 + 2 g]); MFMA s takes l = 8s .. 8s+7.
template <>
struct MoePiece<SPIRAL_TYPE_Q6_K> {
  uint4 l0, l1, h0, h1;
  uint32_t ds2;  // fp16 d (bits 0..15), sc for l < 16 (16..23), sc for l >= 16 (24..31)
  int ls, hs;
  static __device__ __forceinline__ int local(int g, int s, int e) { return 32 * g + 8 * s + e; }
  // sb_row = super-block index (row * nb + sb), h = half, g = group
  __device__ __forceinline__ void load(const uint8_t* we, int64_t tot, int64_t sbi, int h, int g) {
    const uint8_t* ql = we + sbi * 128 + 64 * h + 32 * (g & 1);
    const uint8_t* qh = we + tot * 128 + sbi * 64 + 32 * h;
    l0 = *reinterpret_cast<const uint4*>(ql);
    l1 = *reinterpret_cast<const uint4*>(ql + 16);
    h0 = *reinterpret_cast<const uint4*>(qh);
    h1 = *reinterpret_cast<const uint4*>(qh + 16);
    const uint32_t sc = *reinterpret_cast<const uint16_t*>(we + tot * 192 + sbi * 16 + 8 * h + 2 * g);
    ds2 = *reinterpret_cast<const uint16_t*>(we + tot * 208 + sbi * 2) | (sc << 16);
    ls = (g >> 1) * 4;
    hs = 2 * g;
  }
  __device__ __forceinline__ void zero() { l0 = l1 = h0 = h1 = make_uint4(0u, 0u, 0u, 0u); ds2 = 0u; ls = hs = 0; }
  __device__ __forceinline__ uint4 dequant(int s) const {
    const uint4 L = s < 2 ? l0 : l1, H = s < 2 ? h0 : h1;
    const uint32_t wl0 = (s & 1) ? L.z : L.x, wl1 = (s & 1) ? L.w : L.y;
    const uint32_t wh0 = (s & 1) ? H.z : H.x, wh1 = (s & 1) ? H.w : H.y;
    const float ds = fp16_scale(ds2 & 0xffffu) * static_cast<float>(static_cast<int8_t>(ds2 >> (s < 2 ? 16 : 24)));
    const float off = -32.0f * ds;
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t c = (((i ? wl1 : wl0) >> ls) & 0x0F0F0F0Fu) | ((((i ? wh1 : wh0) >> hs) & 0x03030303u) << 4);
      o[2 * i] = pack_bf16x2(__builtin_fmaf(static_cast<float>(c & 0xffu), ds, off),
                             __builtin_fmaf(static_cast<float>((c >> 8) & 0xffu), ds, off));
      o[2 * i + 1] = pack_bf16x2(__builtin_fmaf(static_cast<float>((c >> 16) & 0xffu), ds, off),
                                 __builtin_fmaf(static_cast<float>(c >> 24), ds, off));
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
  }
};

constexpr int kMoeKC = 1024;                  // k chunk of activations staged in LDS
constexpr int kMoeTok = 16;                   // tokens per pass (one MFMA row block)
constexpr int kMoeAPitch = kMoeKC + 8;        // bf16 per staged row
constexpr int kMoeRing = 4;                   // 128-wide k steps of weights in flight

// Pieces of k step `st` (128 wide) for this lane's row n and group g.
template <int TYPE>
__device__ __forceinline__ void moe_load(MoePiece<TYPE>& pc, const uint8_t* we, int64_t n_rows, int64_t nb,
                                         int64_t n, int64_t k, int64_t st, int g) {
  if constexpr (TYPE == SPIRAL_TYPE_Q6_K) {
    pc.load(we, n_rows * nb, n * nb + (st >> 1), static_cast<int>(st & 1), g);
  } else {
    const int64_t b = 4 * st + g;
    if (32 * b >= k) { pc.zero(); return; }
    pc.load(we, n_rows * nb, n * nb + b);
  }
}

// Stage activations k in [c0, c0 + kMoeKC) of the pass's nt token rows in
// MFMA order: item = 8 consecutive LDS positions (one lane group of one MFMA)
// of one row. Positions past k are zero.
template <int TYPE>
__device__ __forceinline__ void moe_stage(uint16_t* As, const uint16_t* __restrict__ x, const int64_t* xrow, int nt,
                                          int64_t k, int64_t c0, int tid) {
  constexpr int kItems = kMoeKC / 8;
  for (int it = tid; it < nt * kItems; it += 256) {
    const int r = it / kItems, q = it % kItems;
    const int j = q >> 4, s = (q >> 2) & 3, gg = q & 3;
    const int64_t kb = c0 + 128 * j;
    const uint16_t* src = x + xrow[r] + kb;
    const int k0 = MoePiece<TYPE>::local(gg, s, 0), k4 = MoePiece<TYPE>::local(gg, s, 4);
    uint2 lo = make_uint2(0u, 0u), hi = make_uint2(0u, 0u);
    if (kb + k0 < k) lo = *reinterpret_cast<const uint2*>(src + k0);
    if (kb + k4 < k) hi = *reinterpret_cast<const uint2*>(src + k4);
    *reinterpret_cast<uint4*>(&As[r * kMoeAPitch + 8 * q]) = make_uint4(lo.x, lo.y, hi.x, hi.y);
  }
}

template <int TYPE, bool F32_OUT>
__global__ void __launch_bounds__(256) moe_kernel(const uint8_t* __restrict__ w, int64_t expert_stride,
                                                  int64_t n_rows, int64_t k, const uint16_t* __restrict__ x,
                                                  int64_t x_slots, int64_t top_k,
                                                  const int32_t* __restrict__ offsets,
                                                  const int32_t* __restrict__ list, void* __restrict__ y) {
  __shared__ __align__(16) uint16_t As[kMoeTok * kMoeAPitch];
  __shared__ int32_t s_pair[kMoeTok];
  __shared__ int64_t s_xrow[kMoeTok];
  const int64_t e = blockIdx.y;
  const int32_t begin = offsets[e], end = offsets[e + 1];
  if (begin >= end) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4;
  // Rows past n_rows are clamped (their outputs are not stored).
  const int64_t n = static_cast<int64_t>(blockIdx.x) * kMoeBN + 16 * wave + (lane & 15);
  const int64_t nc = min(n, n_rows - 1);
  const uint8_t* we = w + e * expert_stride;
  const int64_t nb = k / block_elems(TYPE);
  const int64_t steps = (k + 127) / 128;
  constexpr int kStepsPerChunk = kMoeKC / 128;

  for (int32_t t0 = begin; t0 < end; t0 += kMoeTok) {
    const int nt = min(kMoeTok, end - t0);
    __syncthreads();
    if (tid < kMoeTok) {
      const int32_t pr = tid < nt ? list[t0 + tid] : -1;
      s_pair[tid] = pr;
      if (pr >= 0) {
        const int64_t t = pr / top_k, slot = pr % top_k;
        s_xrow[tid] = (t * x_slots + slot % x_slots) * k;
      }
    }
    __syncthreads();
    // MFMA rows past nt read row nt - 1; their outputs are dropped.
    const uint16_t* arow = As + min(lane & 15, nt - 1) * kMoeAPitch + 8 * g;
    f32x4_t acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // Weight ring: slot st % kMoeRing holds step st's pieces.
    MoePiece<TYPE> ring[kMoeRing];
#pragma unroll
    for (int i = 0; i < kMoeRing - 1; ++i) moe_load<TYPE>(ring[i], we, n_rows, nb, nc, k, min<int64_t>(i, steps - 1), g);

    for (int64_t s0 = 0; s0 < steps; s0 += kMoeRing) {
#pragma unroll
      for (int d = 0; d < kMoeRing; ++d) {
        const int64_t st = s0 + d;
        if (st >= steps) break;
        if (st % kStepsPerChunk == 0) {
          __syncthreads();
          moe_stage<TYPE>(As, x, s_xrow, nt, k, st * 128, tid);
          __syncthreads();
        }
        moe_load<TYPE>(ring[(d + kMoeRing - 1) % kMoeRing], we, n_rows, nb, nc, k,
                       min<int64_t>(st + kMoeRing - 1, steps - 1), g);
        const int j = static_cast<int>(st % kStepsPerChunk);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const bf16x8_t b = __builtin_bit_cast(bf16x8_t, ring[d].dequant(s));
          const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(arow + 8 * (16 * j + 4 * s));
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
        }
      }
    }

    // acc: lane l holds rows 4 (l / 16) + i (routed pairs) of column l % 16
    // (weight row n).
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int32_t pr = s_pair[4 * g + i];
      if (pr >= 0 && n < n_rows) {
        if constexpr (F32_OUT)
          static_cast<float*>(y)[pr * n_rows + n] = acc[i];
        else
          static_cast<__bf16*>(y)[pr * n_rows + n] = static_cast<__bf16>(acc[i]);
      }
    }
  }
}

}  // namespace

int64_t moe_workspace_bytes(int64_t n_expert, int64_t n_pairs) { return 4 * (n_expert + 1 + n_pairs); }

// Arguments validated by the caller.
int moe(int type, const void* w, int64_t expert_stride, int64_t n_expert, int64_t n_rows, int64_t k,
        const uint16_t* x, int64_t x_slots, const int32_t* ids, int64_t n_tokens, int64_t top_k, void* y,
        int y_type, void* workspace, hipStream_t s) {
  const int64_t n_pairs = n_tokens * top_k;
  int32_t* offsets = static_cast<int32_t*>(workspace);
  int32_t* list = offsets + n_expert + 1;
  const int f32 = y_type == SPIRAL_TYPE_F32;
  hipLaunchKernelGGL(route_kernel, dim3(1), dim3(kRouteThreads), 0, s, ids, static_cast<int32_t>(n_pairs),
                     static_cast<int32_t>(n_expert), offsets, list, y, n_rows, f32);
  if (hipGetLastError() != hipSuccess) return SPIRAL_ERR_HIP;
  const dim3 grid(static_cast<unsigned>(ceil_div(n_rows, kMoeBN)), static_cast<unsigned>(n_expert));
  const uint8_t* W = static_cast<const uint8_t*>(w);
#define SPIRAL_MOE(T)                                                                                    \
  do {                                                                                                   \
    if (f32)                                                                                             \
      hipLaunchKernelGGL((moe_kernel<T, true>), grid, dim3(256), 0, s, W, expert_stride, n_rows, k, x,   \
                         x_slots, top_k, offsets, list, y);                                              \
    else                                                                                                 \
      hipLaunchKernelGGL((moe_kernel<T, false>), grid, dim3(256), 0, s, W, expert_stride, n_rows, k, x,  \
                         x_slots, top_k, offsets, list, y);                                              \
  } while (0)
  if (type == SPIRAL_TYPE_Q4_0) SPIRAL_MOE(SPIRAL_TYPE_Q4_0);
  else if (type == SPIRAL_TYPE_Q8_0) SPIRAL_MOE(SPIRAL_TYPE_Q8_0);
  else SPIRAL_MOE(SPIRAL_TYPE_Q6_K);
#undef SPIRAL_MOE
  return launch_status();
}

}  // namespace spiral
