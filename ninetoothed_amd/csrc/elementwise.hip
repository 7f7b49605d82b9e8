// Elementwise add: out[i] = lhs[i] + rhs[i].
//
// HBM-bound: 3 * n * sizeof(T) bytes per launch.  The contiguous path moves 16 bytes
// per lane per operand (global_load_dwordx4 / global_store_dwordx4) in a grid-stride
// loop sized to fill all 256 CUs; the strided path is a scalar grid-stride loop.
// 16-bit types are added in fp32 and rounded once, which equals the native
// half-precision sum (fp32 carries more than 2p+2 bits for p = 11 and p = 8).
#include "nt_common.h"

namespace nt {

template <typename T>
__global__ __launch_bounds__(256) void add_contig_kernel(const typename elem<T>::storage* __restrict__ a,
                                                         const typename elem<T>::storage* __restrict__ b,
                                                         typename elem<T>::storage* __restrict__ c,
                                                         int64_t n) {
  typedef typename elem<T>::storage S;
  constexpr int V = 16 / sizeof(S);
  const int64_t nvec = n / V;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nvec; i += stride) {
    u32x4 va = *(const u32x4*)(a + i * V);
    u32x4 vb = *(const u32x4*)(b + i * V);
    u32x4 vc;
    const S* pa = (const S*)&va;
    const S* pb = (const S*)&vb;
    S* pc = (S*)&vc;
#pragma unroll
    for (int j = 0; j < V; ++j) pc[j] = elem<T>::from_float(elem<T>::to_float(pa[j]) + elem<T>::to_float(pb[j]));
    __builtin_nontemporal_store(vc, (u32x4*)(c + i * V));
  }
  // Tail (fewer than V elements), handled by the first threads of the grid.
  const int64_t tail = nvec * V;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < n - tail) c[tail + t] = elem<T>::from_float(elem<T>::to_float(a[tail + t]) + elem<T>::to_float(b[tail + t]));
}

template <typename T>
__global__ __launch_bounds__(256) void add_strided_kernel(const typename elem<T>::storage* __restrict__ a, int64_t sa,
                                                          const typename elem<T>::storage* __restrict__ b, int64_t sb,
                                                          typename elem<T>::storage* __restrict__ c, int64_t sc,
                                                          int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    c[i * sc] = elem<T>::from_float(elem<T>::to_float(a[i * sa]) + elem<T>::to_float(b[i * sb]));
}

template <typename T>
static int add_launch(const void* lhs, int64_t sl, const void* rhs, int64_t sr, void* out, int64_t so, int64_t n,
                      hipStream_t stream) {
  typedef typename elem<T>::storage S;
  if (n < 0) return NT_ERR_INVALID;
  if (n == 0) return 0;
  if (!lhs || !rhs || !out) return NT_ERR_INVALID;
  const bool contig = sl == 1 && sr == 1 && so == 1 && ((uintptr_t)lhs % 16 == 0) && ((uintptr_t)rhs % 16 == 0) &&
                      ((uintptr_t)out % 16 == 0);
  constexpr int V = 16 / sizeof(S);
  if (contig) {
    int64_t work = cdiv(n, V);
    int64_t blocks = cdiv(work, 256);
    if (blocks > 256 * 16) blocks = 256 * 16;
    hipLaunchKernelGGL(add_contig_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, stream, (const S*)lhs,
                       (const S*)rhs, (S*)out, n);
  } else {
    int64_t blocks = cdiv(n, 256);
    if (blocks > 256 * 16) blocks = 256 * 16;
    hipLaunchKernelGGL(add_strided_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, stream, (const S*)lhs, sl,
                       (const S*)rhs, sr, (S*)out, so, n);
  }
  return launch_status();
}

}  // namespace nt

extern "C" int nt_add_f32(const void* lhs, int64_t sl, const void* rhs, int64_t sr, void* out, int64_t so, int64_t n,
                          hipStream_t stream) {
  return nt::add_launch<float>(lhs, sl, rhs, sr, out, so, n, stream);
}
extern "C" int nt_add_f16(const void* lhs, int64_t sl, const void* rhs, int64_t sr, void* out, int64_t so, int64_t n,
                          hipStream_t stream) {
  return nt::add_launch<nt::f16_t>(lhs, sl, rhs, sr, out, so, n, stream);
}
extern "C" int nt_add_bf16(const void* lhs, int64_t sl, const void* rhs, int64_t sr, void* out, int64_t so,
                           int64_t n, hipStream_t stream) {
  return nt::add_launch<nt::bf16_t>(lhs, sl, rhs, sr, out, so, n, stream);
}

extern "C" int nt_abi_version(void) { return NT_ABI_VERSION; }
