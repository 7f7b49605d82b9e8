// Row softmax over segments of `block` columns (the application's BLOCK_SIZE).
//
// One 256-lane workgroup per segment.  HBM-bound: each element is read once and
// written once (2 * rows * cols * sizeof(T) bytes).  The segment is held in
// registers between the three phases (max, sum of exp, scale), so nothing is
// re-read; reductions are wave64 butterflies plus one LDS exchange across the four
// waves.  exp(x) is computed as exp2(x * log2 e) on the hardware v_exp_f32.
// Segments longer than the register path holds use a two-sweep kernel: an online
// (max, sum) sweep, then a scaling sweep; segments of at most a few vectors per lane of
// one wave use a kernel that gives each segment a group of lanes.
#include "nt_common.h"

namespace nt {

constexpr int SM_THREADS = 256;
constexpr float LOG2E = 1.4426950408889634f;

__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * LOG2E); }

template <int NW>
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}

template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r += red[i];
  __syncthreads();
  return r;
}

// Register path: NT lanes per workgroup, each owning VPT vectors of V elements.
template <typename T, int VPT, bool VEC, int NT = SM_THREADS>
__global__ __launch_bounds__(NT) void softmax_reg_kernel(const typename elem<T>::storage* __restrict__ x,
                                                                 int64_t xs, typename elem<T>::storage* __restrict__ y,
                                                                 int64_t ys, int64_t cols, int64_t block,
                                                                 int64_t segs_per_row) {
  typedef typename elem<T>::storage S;
  constexpr int V = 16 / sizeof(S);
  __shared__ float red[NT / 64];
  const int64_t seg = blockIdx.x;
  const int64_t row = seg / segs_per_row;
  const int64_t c0 = (seg % segs_per_row) * block;
  const int64_t len = (cols - c0 < block) ? (cols - c0) : block;
  const S* xr = x + row * xs + c0;
  S* yr = y + row * ys + c0;

  float v[VPT][V];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int64_t e0 = ((int64_t)j * NT + threadIdx.x) * V;
    if (VEC && e0 + V <= len) {
      u32x4 raw = *(const u32x4*)(xr + e0);  // plain load: nontemporal loads cost ~8% here
      const S* p = (const S*)&raw;
#pragma unroll
      for (int u = 0; u < V; ++u) v[j][u] = elem<T>::to_float(p[u]);
    } else {
#pragma unroll
      for (int u = 0; u < V; ++u) v[j][u] = (e0 + u < len) ? elem<T>::to_float(xr[e0 + u]) : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < V; ++u) mx = fmaxf(mx, v[j][u]);
  }
  mx = block_max<NT / 64>(mx, red);
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
#pragma unroll
    for (int u = 0; u < V; ++u) {
      v[j][u] = fast_exp(v[j][u] - mx);
      sum += v[j][u];
    }
  }
  sum = block_sum<NT / 64>(sum, red);
  const float inv = 1.0f / sum;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int64_t e0 = ((int64_t)j * NT + threadIdx.x) * V;
    if (VEC && e0 + V <= len) {
      u32x4 raw;
      S* p = (S*)&raw;
#pragma unroll
      for (int u = 0; u < V; ++u) p[u] = elem<T>::from_float(v[j][u] * inv);
      __builtin_nontemporal_store(raw, (u32x4*)(yr + e0));
    } else {
#pragma unroll
      for (int u = 0; u < V; ++u)
        if (e0 + u < len) yr[e0 + u] = elem<T>::from_float(v[j][u] * inv);
    }
  }
}

// Segment layout for the lane-group and two-sweep kernels: with VEC (x and y share their
// 16-byte phase at every segment start) the first `head` elements (up to the first 16-byte
// boundary of x) are single elements, the rest 16-byte vectors from that boundary, the
// last partial vector single elements again; so rows whose length is no multiple of 16
// bytes still move in whole vectors.  Without VEC, head = 0 and every element is single.
template <typename S, bool VEC>
__device__ __forceinline__ int seg_head(const S* xr, int64_t len) {
  if constexpr (!VEC) return 0;
  const int h = (int)(((16 - ((uintptr_t)xr & 15)) & 15) / sizeof(S));
  return len < h ? (int)len : h;
}

// Short segments: a group of LPR lanes (a power of two, at most a wave) per segment, each
// lane holding VPT vectors of V elements (and up to HN head elements: the head has at most
// V - 1 elements, strided over the group's lanes), so a 256-lane workgroup
// takes 256 / LPR segments (one per 16 lanes for 128 fp16 columns) instead of leaving most
// of its lanes idle.  The reductions are butterflies inside the group.
template <int LPR>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
template <typename T, int LPR, int VPT, bool VEC>
__global__ __launch_bounds__(SM_THREADS) void softmax_rows_kernel(const typename elem<T>::storage* __restrict__ x,
                                                                  int64_t xs, typename elem<T>::storage* __restrict__ y,
                                                                  int64_t ys, int64_t cols, int64_t block,
                                                                  int64_t segs_per_row, int64_t segs) {
  typedef typename elem<T>::storage S;
  constexpr int V = 16 / sizeof(S);
  const int64_t seg = (int64_t)blockIdx.x * (SM_THREADS / LPR) + threadIdx.x / LPR;
  if (seg >= segs) return;  // whole groups leave together: the butterflies stay inside a group
  const int gl = threadIdx.x % LPR;
  const int64_t row = seg / segs_per_row;
  const int64_t c0 = (seg % segs_per_row) * block;
  const int64_t len = (cols - c0 < block) ? (cols - c0) : block;
  const S* xr = x + row * xs + c0;
  S* yr = y + row * ys + c0;
  const int head = seg_head<S, VEC>(xr, len);
  const S* xb = xr + head;
  S* yb = yr + head;
  const int64_t blen = len - head;
  constexpr int HN = (V - 1 + LPR - 1) / LPR;  // head elements gl, gl + LPR, ... per lane
  float hv[HN];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < HN; ++i) {
    const int e = gl + i * LPR;
    hv[i] = e < head ? elem<T>::to_float(xr[e]) : -INFINITY;
    mx = fmaxf(mx, hv[i]);
  }
  float v[VPT][V];
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int64_t e0 = ((int64_t)j * LPR + gl) * V;
    if (VEC && e0 + V <= blen) {
      u32x4 raw = *(const u32x4*)(xb + e0);
      const S* p = (const S*)&raw;
#pragma unroll
      for (int u = 0; u < V; ++u) v[j][u] = elem<T>::to_float(p[u]);
    } else {
#pragma unroll
      for (int u = 0; u < V; ++u) v[j][u] = (e0 + u < blen) ? elem<T>::to_float(xb[e0 + u]) : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < V; ++u) mx = fmaxf(mx, v[j][u]);
  }
  mx = group_max<LPR>(mx);
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < HN; ++i) {
    hv[i] = fast_exp(hv[i] - mx);
    if (gl + i * LPR < head) sum += hv[i];
  }
#pragma unroll
  for (int j = 0; j < VPT; ++j)
#pragma unroll
    for (int u = 0; u < V; ++u) {
      v[j][u] = fast_exp(v[j][u] - mx);
      sum += v[j][u];
    }
  const float inv = 1.0f / group_sum<LPR>(sum);
#pragma unroll
  for (int i = 0; i < HN; ++i)
    if (gl + i * LPR < head) yr[gl + i * LPR] = elem<T>::from_float(hv[i] * inv);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int64_t e0 = ((int64_t)j * LPR + gl) * V;
    if (VEC && e0 + V <= blen) {
      u32x4 raw;
      S* p = (S*)&raw;
#pragma unroll
      for (int u = 0; u < V; ++u) p[u] = elem<T>::from_float(v[j][u] * inv);
      __builtin_nontemporal_store(raw, (u32x4*)(yb + e0));
    } else {
#pragma unroll
      for (int u = 0; u < V; ++u)
        if (e0 + u < blen) yb[e0 + u] = elem<T>::from_float(v[j][u] * inv);
    }
  }
}

// Long segments: an online (max, sum) sweep, then a scaling sweep.  Each lane takes U
// vectors of V elements per step with all their loads issued first, so a workgroup keeps
// NT * U * 16 bytes in flight (128 KiB with 1024 lanes): with few segments (few
// workgroups) each one must fetch at a whole CU's rate.  Per vector one rescale of the
// running sum (to the vector's max) and V exponentials.
template <typename T, int NT, bool VEC>
__global__ __launch_bounds__(NT) void softmax_long_kernel(const typename elem<T>::storage* __restrict__ x,
                                                          int64_t xs, typename elem<T>::storage* __restrict__ y,
                                                          int64_t ys, int64_t cols, int64_t block,
                                                          int64_t segs_per_row) {
  typedef typename elem<T>::storage S;
  constexpr int V = 16 / sizeof(S), U = 8;
  __shared__ float red[NT / 64];
  const int64_t seg = blockIdx.x;
  const int64_t row = seg / segs_per_row;
  const int64_t c0 = (seg % segs_per_row) * block;
  const int64_t len = (cols - c0 < block) ? (cols - c0) : block;
  const S* xr = x + row * xs + c0;
  S* yr = y + row * ys + c0;
  const int head = seg_head<S, VEC>(xr, len);
  const S* xb = xr + head;
  S* yb = yr + head;
  const int64_t blen = len - head;
  auto load = [&](int64_t e0, float (&v)[V]) {
    if (VEC && e0 + V <= blen) {
      u32x4 raw = *(const u32x4*)(xb + e0);
      const S* p = (const S*)&raw;
#pragma unroll
      for (int u = 0; u < V; ++u) v[u] = elem<T>::to_float(p[u]);
    } else {
#pragma unroll
      for (int u = 0; u < V; ++u) v[u] = (e0 + u < blen) ? elem<T>::to_float(xb[e0 + u]) : -INFINITY;
    }
  };
  constexpr int64_t STEP = (int64_t)NT * V * U;
  // The head element of this lane (if any) starts the running (max, sum).
  const float hv = (int)threadIdx.x < head ? elem<T>::to_float(xr[threadIdx.x]) : -INFINITY;
  float m = hv, s = hv == -INFINITY ? 0.f : 1.f;
  for (int64_t base = 0; base < blen; base += STEP) {
    float v[U][V];
#pragma unroll
    for (int j = 0; j < U; ++j) load(base + ((int64_t)j * NT + threadIdx.x) * V, v[j]);
#pragma unroll
    for (int j = 0; j < U; ++j) {
      float vm = v[j][0];
#pragma unroll
      for (int u = 1; u < V; ++u) vm = fmaxf(vm, v[j][u]);
      if (vm != -INFINITY) {  // a vector of -inf (or past the end) adds nothing
        const float nm = fmaxf(m, vm);
        s = (m == -INFINITY) ? 0.f : s * fast_exp(m - nm);
        m = nm;
#pragma unroll
        for (int u = 0; u < V; ++u) s += fast_exp(v[j][u] - m);
      }
    }
  }
  // Combine per-lane (m, s) pairs: rescale every partial sum to the block max.
  const float gm = block_max<NT / 64>(m, red);
  const float part = (m == -INFINITY) ? 0.f : s * fast_exp(m - gm);
  const float gs = block_sum<NT / 64>(part, red);
  const float inv = 1.0f / gs;
  if ((int)threadIdx.x < head) yr[threadIdx.x] = elem<T>::from_float(fast_exp(hv - gm) * inv);
  for (int64_t base = 0; base < blen; base += STEP) {
    float v[U][V];
#pragma unroll
    for (int j = 0; j < U; ++j) load(base + ((int64_t)j * NT + threadIdx.x) * V, v[j]);
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int64_t e0 = base + ((int64_t)j * NT + threadIdx.x) * V;
      if (VEC && e0 + V <= blen) {
        u32x4 raw;
        S* p = (S*)&raw;
#pragma unroll
        for (int u = 0; u < V; ++u) p[u] = elem<T>::from_float(fast_exp(v[j][u] - gm) * inv);
        __builtin_nontemporal_store(raw, (u32x4*)(yb + e0));
      } else {
#pragma unroll
        for (int u = 0; u < V; ++u)
          if (e0 + u < blen) yb[e0 + u] = elem<T>::from_float(fast_exp(v[j][u] - gm) * inv);
      }
    }
  }
}

// Any strides and any pair of element types (the reference passes strides to its kernel and
// its store casts to the output's type): one 256-lane workgroup per segment, element-wise
// loads at the column stride, U elements per lane in flight, an online (max, sum) sweep,
// then a sweep that recomputes exp(x - max) / sum and stores it in the output's type.
template <typename Ti, typename To>
__global__ __launch_bounds__(SM_THREADS) void softmax_any_kernel(const typename elem<Ti>::storage* __restrict__ x,
                                                                 int64_t xs, int64_t xcs,
                                                                 typename elem<To>::storage* __restrict__ y,
                                                                 int64_t ys, int64_t ycs, int64_t cols, int64_t block,
                                                                 int64_t segs_per_row) {
  constexpr int U = 8;
  constexpr int64_t STEP = (int64_t)SM_THREADS * U;
  __shared__ float red[SM_THREADS / 64];
  const int64_t seg = blockIdx.x;
  const int64_t row = seg / segs_per_row;
  const int64_t c0 = (seg % segs_per_row) * block;
  const int64_t len = (cols - c0 < block) ? (cols - c0) : block;
  const typename elem<Ti>::storage* xr = x + row * xs + c0 * xcs;
  typename elem<To>::storage* yr = y + row * ys + c0 * ycs;
  float m = -INFINITY, s = 0.f;
  for (int64_t base = 0; base < len; base += STEP) {
    float v[U];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int64_t e = base + (int64_t)j * SM_THREADS + threadIdx.x;
      v[j] = e < len ? elem<Ti>::to_float(xr[e * xcs]) : -INFINITY;
    }
    float vm = v[0];
#pragma unroll
    for (int j = 1; j < U; ++j) vm = fmaxf(vm, v[j]);
    if (vm != -INFINITY) {
      const float nm = fmaxf(m, vm);
      s = (m == -INFINITY) ? 0.f : s * fast_exp(m - nm);
      m = nm;
#pragma unroll
      for (int j = 0; j < U; ++j) s += fast_exp(v[j] - m);
    }
  }
  const float gm = block_max<SM_THREADS / 64>(m, red);
  const float part = (m == -INFINITY) ? 0.f : s * fast_exp(m - gm);
  const float inv = 1.0f / block_sum<SM_THREADS / 64>(part, red);
  for (int64_t base = 0; base < len; base += STEP) {
    float v[U];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int64_t e = base + (int64_t)j * SM_THREADS + threadIdx.x;
      v[j] = e < len ? elem<Ti>::to_float(xr[e * xcs]) : 0.f;
    }
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int64_t e = base + (int64_t)j * SM_THREADS + threadIdx.x;
      if (e < len) yr[e * ycs] = elem<To>::from_float(fast_exp(v[j] - gm) * inv);
    }
  }
}

template <typename Ti, typename To>
static void softmax_any_launch(const void* x, int64_t xs, int64_t xcs, void* y, int64_t ys, int64_t ycs, int64_t cols,
                               int64_t block, int64_t segs_per_row, int64_t segs, hipStream_t stream) {
  hipLaunchKernelGGL((softmax_any_kernel<Ti, To>), dim3((unsigned)segs), dim3(SM_THREADS), 0, stream,
                     (const typename elem<Ti>::storage*)x, xs, xcs, (typename elem<To>::storage*)y, ys, ycs, cols,
                     block, segs_per_row);
}

// config: 0 = the lane-group kernel for segments of at most 4 vectors per lane of a wave,
// else the four-wave register path when the segment fits it (16 vectors of 16 bytes per
// lane at most), else the two-sweep kernel; 1 = four-wave register path; 2 = eight-wave
// register path; 3 = one-wave register path; 4 = two-sweep kernel; 5 = lane-group kernel
// 6 = the any-strides kernel (the only one for a column stride other than 1, so config 0
// takes it then) (the reference's auto-tuner times num_warps 4, 8, 1:
// src/ninetoothed/backends/triton.py:151-155).  A forced kernel whose conditions do not
// hold returns NT_ERR_INVALID unlaunched.
template <typename T>
static int softmax_launch(const void* x, int64_t xs, int64_t xcs, void* y, int64_t ys, int64_t ycs, int64_t rows,
                          int64_t cols, int64_t block, hipStream_t stream, int config = 0) {
  typedef typename elem<T>::storage S;
  constexpr int V = 16 / sizeof(S);
  if (config < 0 || config > 6) return NT_ERR_INVALID;
  if (rows < 0 || cols < 0 || block <= 0) return NT_ERR_INVALID;
  if (rows == 0 || cols == 0) return 0;
  if (!x || !y) return NT_ERR_INVALID;
  const int64_t segs_per_row = cdiv(cols, block);
  const int64_t segs = rows * segs_per_row;
  if (segs > 0x7fffffffLL) return NT_ERR_INVALID;
  const bool unit = cols <= 1 || (xcs == 1 && ycs == 1);
  if (config == 6 || (config == 0 && !unit)) {
    softmax_any_launch<T, T>(x, xs, xcs, y, ys, ycs, cols, block, segs_per_row, segs, stream);
    return launch_status();
  }
  if (!unit) return NT_ERR_INVALID;
  const int64_t len = block < cols ? block : cols;
  const bool vec = ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 16 == 0) && ((xs * (int64_t)sizeof(S)) % 16 == 0 || rows == 1) &&
                   ((ys * (int64_t)sizeof(S)) % 16 == 0 || rows == 1) &&
                   ((block * (int64_t)sizeof(S)) % 16 == 0 || segs_per_row == 1);
  // The lane-group and two-sweep kernels need only x and y in the same 16-byte phase at
  // every segment start (they split off a head up to the boundary).
  const bool coal = ((uintptr_t)x % sizeof(S) == 0) && ((uintptr_t)y % sizeof(S) == 0) &&
                    (((uintptr_t)x - (uintptr_t)y) % 16 == 0) && (((xs - ys) * (int64_t)sizeof(S)) % 16 == 0 || rows == 1);
  const dim3 grid((unsigned)segs);
  const S* xp = (const S*)x;
  S* yp = (S*)y;
  // Launch the register path with NT lanes and the smallest VPT that holds the segment (up
  // to 16 with 16-byte accesses, 8 with element-wise ones, whose per-element bounds checks
  // would spill beyond); false when none does.
  auto reg = [&](auto nt_c) {
    constexpr int NT = decltype(nt_c)::value;
    bool done = false;
    static_for<0, 5>([&](auto e_c) {
      constexpr int VPT = 1 << decltype(e_c)::value;
      if (done || len > (int64_t)NT * V * VPT) return;
      if (vec) {
        hipLaunchKernelGGL((softmax_reg_kernel<T, VPT, true, NT>), grid, dim3(NT), 0, stream, xp, xs, yp, ys, cols,
                           block, segs_per_row);
        done = true;
      } else if constexpr (VPT <= 8) {
        hipLaunchKernelGGL((softmax_reg_kernel<T, VPT, false, NT>), grid, dim3(NT), 0, stream, xp, xs, yp, ys, cols,
                           block, segs_per_row);
        done = true;
      }
    });
    return done;
  };
  // Segments of at most 4 vectors per lane of one wave: a group of LPR lanes per segment
  // (LPR the smallest power of two with LPR * VPT * V >= len, VPT 1, 2 or 4).
  auto groups = [&]() {
    bool done = false;
    static_for<0, 7>([&](auto l_c) {
      constexpr int LPR = 1 << decltype(l_c)::value;
      static_for<0, 3>([&](auto p_c) {
        constexpr int VPT = 1 << decltype(p_c)::value;
        if constexpr (VPT == 1 || LPR == 64) {
          if (done || len > (int64_t)LPR * V * VPT) return;
          const dim3 g2((unsigned)cdiv(segs, SM_THREADS / LPR));
          if (coal)
            hipLaunchKernelGGL((softmax_rows_kernel<T, LPR, VPT, true>), g2, dim3(SM_THREADS), 0, stream, xp, xs, yp,
                               ys, cols, block, segs_per_row, segs);
          else
            hipLaunchKernelGGL((softmax_rows_kernel<T, LPR, VPT, false>), g2, dim3(SM_THREADS), 0, stream, xp, xs,
                               yp, ys, cols, block, segs_per_row, segs);
          done = true;
        }
      });
    });
    return done;
  };
  // The two-sweep kernel: 1024 lanes per segment when there are too few segments to give
  // every CU two workgroups, else 256.
  auto sweep = [&]() {
    if (segs < 512) {
      if (coal)
        hipLaunchKernelGGL((softmax_long_kernel<T, 1024, true>), grid, dim3(1024), 0, stream, xp, xs, yp, ys, cols,
                           block, segs_per_row);
      else
        hipLaunchKernelGGL((softmax_long_kernel<T, 1024, false>), grid, dim3(1024), 0, stream, xp, xs, yp, ys, cols,
                           block, segs_per_row);
    } else if (coal) {
      hipLaunchKernelGGL((softmax_long_kernel<T, SM_THREADS, true>), grid, dim3(SM_THREADS), 0, stream, xp, xs, yp,
                         ys, cols, block, segs_per_row);
    } else {
      hipLaunchKernelGGL((softmax_long_kernel<T, SM_THREADS, false>), grid, dim3(SM_THREADS), 0, stream, xp, xs, yp,
                         ys, cols, block, segs_per_row);
    }
  };
  using W4 = std::integral_constant<int, 256>;
  using W8 = std::integral_constant<int, 512>;
  using W1 = std::integral_constant<int, 64>;
  if (config == 0) {
    if (len > (int64_t)4 * 64 * V || !groups())
      if (!reg(W4{})) sweep();
  } else if (config == 4) {
    sweep();
  } else if (config == 5) {
    if (!groups()) return NT_ERR_INVALID;
  } else if ((config == 1 && !reg(W4{})) || (config == 2 && !reg(W8{})) || (config == 3 && !reg(W1{}))) {
    return NT_ERR_INVALID;
  }
  return launch_status();
}

// Input and output of any two element types: same types take softmax_launch's kernels,
// others the any-strides kernel.
template <typename Ti>
static int softmax_cast_to(const void* x, int64_t xs, int64_t xcs, void* y, int y_dtype, int64_t ys, int64_t ycs,
                           int64_t rows, int64_t cols, int64_t block, hipStream_t stream) {
  if (y_dtype == elem<Ti>::code) return softmax_launch<Ti>(x, xs, xcs, y, ys, ycs, rows, cols, block, stream);
  if (!valid_dtype(y_dtype) || rows < 0 || cols < 0 || block <= 0) return NT_ERR_INVALID;
  if (rows == 0 || cols == 0) return 0;
  if (!x || !y) return NT_ERR_INVALID;
  const int64_t segs_per_row = cdiv(cols, block);
  const int64_t segs = rows * segs_per_row;
  if (segs > 0x7fffffffLL) return NT_ERR_INVALID;
  if (y_dtype == NT_DTYPE_F32)
    softmax_any_launch<Ti, float>(x, xs, xcs, y, ys, ycs, cols, block, segs_per_row, segs, stream);
  else if (y_dtype == NT_DTYPE_F16)
    softmax_any_launch<Ti, f16_t>(x, xs, xcs, y, ys, ycs, cols, block, segs_per_row, segs, stream);
  else
    softmax_any_launch<Ti, bf16_t>(x, xs, xcs, y, ys, ycs, cols, block, segs_per_row, segs, stream);
  return launch_status();
}

}  // namespace nt

extern "C" int nt_softmax_cast(const void* x, int x_dtype, int64_t xs, int64_t xcs, void* y, int y_dtype, int64_t ys,
                               int64_t ycs, int64_t rows, int64_t cols, int64_t block, hipStream_t stream) {
  if (x_dtype == NT_DTYPE_F32) return nt::softmax_cast_to<float>(x, xs, xcs, y, y_dtype, ys, ycs, rows, cols, block, stream);
  if (x_dtype == NT_DTYPE_F16)
    return nt::softmax_cast_to<nt::f16_t>(x, xs, xcs, y, y_dtype, ys, ycs, rows, cols, block, stream);
  if (x_dtype == NT_DTYPE_BF16)
    return nt::softmax_cast_to<nt::bf16_t>(x, xs, xcs, y, y_dtype, ys, ycs, rows, cols, block, stream);
  return NT_ERR_INVALID;
}

extern "C" int nt_softmax_f32(const void* x, int64_t xs, int64_t xcs, void* y, int64_t ys, int64_t ycs, int64_t rows,
                              int64_t cols, int64_t block, hipStream_t stream) {
  return nt::softmax_launch<float>(x, xs, xcs, y, ys, ycs, rows, cols, block, stream);
}
extern "C" int nt_softmax_f16(const void* x, int64_t xs, int64_t xcs, void* y, int64_t ys, int64_t ycs, int64_t rows,
                              int64_t cols, int64_t block, hipStream_t stream) {
  return nt::softmax_launch<nt::f16_t>(x, xs, xcs, y, ys, ycs, rows, cols, block, stream);
}
extern "C" int nt_softmax_bf16(const void* x, int64_t xs, int64_t xcs, void* y, int64_t ys, int64_t ycs, int64_t rows,
                               int64_t cols, int64_t block, hipStream_t stream) {
  return nt::softmax_launch<nt::bf16_t>(x, xs, xcs, y, ys, ycs, rows, cols, block, stream);
}
extern "C" int nt_softmax_config_f32(const void* x, int64_t xs, int64_t xcs, void* y, int64_t ys, int64_t ycs,
                                     int64_t rows, int64_t cols, int64_t block, hipStream_t stream, int config) {
  return nt::softmax_launch<float>(x, xs, xcs, y, ys, ycs, rows, cols, block, stream, config);
}
extern "C" int nt_softmax_config_f16(const void* x, int64_t xs, int64_t xcs, void* y, int64_t ys, int64_t ycs,
                                     int64_t rows, int64_t cols, int64_t block, hipStream_t stream, int config) {
  return nt::softmax_launch<nt::f16_t>(x, xs, xcs, y, ys, ycs, rows, cols, block, stream, config);
}
extern "C" int nt_softmax_config_bf16(const void* x, int64_t xs, int64_t xcs, void* y, int64_t ys, int64_t ycs,
                                      int64_t rows, int64_t cols, int64_t block, hipStream_t stream, int config) {
  return nt::softmax_launch<nt::bf16_t>(x, xs, xcs, y, ys, ycs, rows, cols, block, stream, config);
}
