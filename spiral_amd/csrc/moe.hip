// Grouped dequant-GEMM for mixture-of-experts (ggml MUL_MAT_ID with
// quantized, expert-stacked weights).
//
// Two launches on the caller's stream:
//  1. route_kernel (one workgroup): a counting sort of the (token, slot)
//     pairs by expert id into per-expert lists in the caller's workspace;
//     pairs with an out-of-range id get a zero output row.
//  2. moe_kernel: workgroup (n-tile, expert) streams that expert's BN weight
//     rows once and multiplies them against every token routed to it, 16
//     tokens per MFMA row tile, up to 64 tokens per pass. Each expert's
//     weights are therefore read from HBM once per call, which is what bounds
//     this op at decode batch sizes (a few tokens per expert).
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
constexpr int kMoeBN = 64, kMoeBK = 64, kMoeTok = 64;
constexpr int kMoeLdsK = kMoeBK + 8;

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

template <int TYPE, bool F32_OUT>
__global__ void __launch_bounds__(256) moe_kernel(const uint8_t* __restrict__ w, int64_t expert_stride,
                                                  int64_t n_rows, int64_t k, const uint16_t* __restrict__ x,
                                                  int64_t x_slots, int64_t top_k,
                                                  const int32_t* __restrict__ offsets,
                                                  const int32_t* __restrict__ list, void* __restrict__ y) {
  __shared__ __align__(16) uint16_t As[kMoeTok * kMoeLdsK];
  __shared__ __align__(16) uint16_t Bs[kMoeBN * kMoeLdsK];
  __shared__ int32_t s_pair[kMoeTok];
  const int64_t e = blockIdx.y;
  const int32_t begin = offsets[e], end = offsets[e + 1];
  if (begin >= end) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kMoeBN;
  const uint8_t* we = w + e * expert_stride;
  const int64_t nb = k / block_elems(TYPE);

  for (int32_t t0 = begin; t0 < end; t0 += kMoeTok) {
    const int nt = min(kMoeTok, end - t0);
    const int chunks = (nt + 15) / 16;
    __syncthreads();
    if (tid < kMoeTok) s_pair[tid] = tid < nt ? list[t0 + tid] : -1;
    __syncthreads();
    f32x4_t acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    for (int64_t k0 = 0; k0 < k; k0 += kMoeBK) {
      // Token rows (gathered): 64 tokens x 64 k as 16-byte pieces.
#pragma unroll
      for (int it = 0; it < (kMoeTok * kMoeBK / 8) / 256; ++it) {
        const int i = tid + 256 * it;
        const int r = i >> 3, c = i & 7;
        const int64_t gk = k0 + 8 * c;
        const int32_t p = s_pair[r];
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (p >= 0 && gk < k) {
          const int64_t t = p / top_k, slot = p % top_k;
          v = *reinterpret_cast<const uint4*>(x + (t * x_slots + slot % x_slots) * k + gk);
        }
        *reinterpret_cast<uint4*>(&As[r * kMoeLdsK + 8 * c]) = v;
      }
      // Expert weight rows n0 .. n0 + 63, dequantized exactly.
#pragma unroll
      for (int it = 0; it < (kMoeBN * kMoeBK / 8) / 256; ++it) {
        const int i = tid + 256 * it;
        const int r = i >> 3, c = i & 7;
        const int64_t gn = n0 + r, g = (k0 >> 3) + c;
        float v[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        if (gn < n_rows && 8 * g < k) dequant8<TYPE>(we, n_rows, nb, gn, g, v);
        *reinterpret_cast<uint4*>(&Bs[r * kMoeLdsK + 8 * c]) =
            make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                       pack_bf16x2(v[6], v[7]));
      }
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < kMoeBK; kk += 32) {
        const int kq = kk + 8 * (lane >> 4);
        const bf16x8_t b = *reinterpret_cast<const bf16x8_t*>(&Bs[(wave * 16 + (lane & 15)) * kMoeLdsK + kq]);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (c < chunks) {
            const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(&As[(16 * c + (lane & 15)) * kMoeLdsK + kq]);
            acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[c], 0, 0, 0);
          }
        }
      }
      __syncthreads();
    }

    const int64_t gn = n0 + wave * 16 + (lane & 15);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (c >= chunks) break;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = 16 * c + 4 * (lane >> 4) + q;
        const int32_t p = s_pair[r];
        if (p >= 0 && gn < n_rows) {
          if constexpr (F32_OUT)
            static_cast<float*>(y)[p * n_rows + gn] = acc[c][q];
          else
            static_cast<__bf16*>(y)[p * n_rows + gn] = static_cast<__bf16>(acc[c][q]);
        }
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
