// Fused attention forward (online softmax in base 2) on the MFMA tile core.
//
// One workgroup per (batch, head, block of 128 queries); four waves, each owning 32
// queries.  Keys and values stream through LDS in tiles of 64.  The kernel works in
// the transposed frame:
//   S^T = K . Q^T      (v_mfma_f32_32x32x16: a = K rows from LDS, b = Q^T held in
//                       registers for the whole key loop)
//   O^T += V^T . P^T   (a = V^T rows from LDS, b = P^T taken straight from the S^T
//                       accumulators after exp2 and rounding)
// In the 32x32 accumulator layout a lane holds one query (lane % 32) and 16 keys, so
// the per-query max and sum need a single cross-lane exchange (lane ^ 32), the
// rescale by alpha is a per-lane scalar, and P^T never leaves registers: for the k
// slice t of 16 keys, slot s of a lane is accumulator register 8*(t%2) + s of key
// block t/2, i.e. key 16t + (s/4)*8 + (lane/32)*4 + s%4; V^T is fetched with the same
// key order (two 8-byte LDS reads per fragment).
// K tiles are stored [d-half][key][64 d] and V^T tiles [d][64 keys], both with the
// 16-byte chunk swizzle of the MFMA core; V is transposed 8x8 in registers on its way
// from HBM.  The next key tile is fetched into registers during the current tile's
// math.  Causal launches stop at the last key tile a query block can see, and the
// heaviest query blocks are launched first.
// MFMA-bound: 4 * B * H * Sq * Sk * D flops per launch (half of that when causal).
#include "mfma_core.h"

namespace nt {

constexpr int AT_BM = 128;  // queries per workgroup
constexpr int AT_BN = 64;   // keys per tile
constexpr int AT_THREADS = 256;

struct AttnArgs {
  const void *q, *k, *v;
  void* o;
  int64_t qs[4], ks[4], vs[4], os[4];
  int64_t B, H, Sq, Sk, D;
  float q_scale;
  int causal, o_dtype, q_blocks;
};

// Workgroup id -> (query block, batch*head).  The dispatcher hands ids to the 8 XCDs
// round-robin (id % 8), each XCD with its own L2.  When B*H divides by 8, XCD x owns the
// heads [x*BH/8, (x+1)*BH/8): non-causal launches walk them head by head (a head's K and V
// stay hot in that L2 while its query blocks run); causal launches walk them in groups of
// four heads, heaviest query block first within a group (longest job first, with only
// about four heads' K and V in flight per L2: ungrouped, the causal launch re-fetched
// K/V from HBM 3.4 times over).  Otherwise: heaviest first, heads fastest.
__device__ __forceinline__ void block_order(const AttnArgs& g, int64_t id, int& qb, int64_t& bh) {
  const int64_t BH = g.B * g.H;
  const int64_t nq = g.q_blocks;
  if (BH % 8 == 0) {
    const int64_t per_xcd = BH / 8;
    const int64_t x = id % 8, local = id / 8;
    if (g.causal) {
      constexpr int HG = 4;  // heads per group
      if (per_xcd % HG == 0) {
        const int64_t grp = local / (HG * nq), within = local % (HG * nq);
        qb = (int)(nq - 1 - within / HG);
        bh = x * per_xcd + grp * HG + within % HG;
      } else {
        qb = (int)(nq - 1 - local / per_xcd);
        bh = x * per_xcd + local % per_xcd;
      }
    } else {
      qb = (int)(local % nq);
      bh = x * per_xcd + local / nq;
    }
    return;
  }
  qb = (int)(nq - 1 - id / BH);
  bh = id % BH;
}

template <typename T, int DM, bool KVEC>  // DM = padded head dim (64 or 128)
__device__ __forceinline__ void attention_body(const AttnArgs& g) {
  typedef typename mfma_traits<T>::frag frag;
  constexpr int DH = DM / 64;  // 64-wide d halves
  constexpr int DSUB = DM / 16;
  constexpr int DBLK = DM / 32;
  // K tile [d-half][key][64 d] (chunk-swizzled) and V^T tile [d][64 keys + 4 pad]; the
  // pad shifts consecutive d rows by two banks so that the 8-byte fragment reads of 16
  // rows hit 32 distinct banks.  Reused at the end to stage the output.
  constexpr int VT_STRIDE = TILE_K + 4;
  constexpr int SMEM = (DH * AT_BN * TILE_K + DM * VT_STRIDE) > (4 * 32 * 65 * 2) ? (DH * AT_BN * TILE_K + DM * VT_STRIDE)
                                                                                   : (4 * 32 * 65 * 2);
  __shared__ __attribute__((aligned(16))) uint16_t smem[SMEM];
  uint16_t* sK = smem;
  uint16_t* sVt = smem + DH * AT_BN * TILE_K;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5;
  int qb;
  int64_t bh;
  block_order(g, blockIdx.x, qb, bh);
  const int64_t b = bh / g.H, h = bh % g.H;
  const int64_t q0 = (int64_t)qb * AT_BM;
  const uint16_t* Q = (const uint16_t*)g.q + b * g.qs[0] + h * g.qs[1];
  const uint16_t* K = (const uint16_t*)g.k + b * g.ks[0] + h * g.ks[1];
  const uint16_t* V = (const uint16_t*)g.v + b * g.vs[0] + h * g.vs[1];

  // Q^T fragments of this lane's query, pre-scaled and rounded to the input type.
  const int64_t qpos = q0 + wave * 32 + (lane & 31);
  frag qf[DSUB];
#pragma unroll
  for (int dd = 0; dd < DSUB; ++dd) {
    uint16_t tmp[8];
    if (KVEC) {  // unit d-stride and 16-byte aligned rows (checked at launch)
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (qpos < g.Sq) raw = *(const u32x4*)(Q + qpos * g.qs[2] + dd * 16 + half * 8);
      const uint16_t* h = (const uint16_t*)&raw;
#pragma unroll
      for (int u = 0; u < 8; ++u) tmp[u] = elem<T>::from_float(elem<T>::to_float(h[u]) * g.q_scale);
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t d = dd * 16 + half * 8 + u;
        float x = 0.f;
        if (qpos < g.Sq && d < g.D) x = elem<T>::to_float(Q[qpos * g.qs[2] + d * g.qs[3]]) * g.q_scale;
        tmp[u] = elem<T>::from_float(x);
      }
    }
    qf[dd] = __builtin_bit_cast(frag, *(const u32x4*)tmp);
  }

  floatx16 o_acc[DBLK];
#pragma unroll
  for (int i = 0; i < DBLK; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[i][r] = 0.f;
  float m_i = -INFINITY, l_i = 1.0f;

  int64_t nkt = cdiv(g.Sk, AT_BN);
  if (g.causal) {
    const int64_t last = (q0 + AT_BM - 1) / AT_BN + 1;
    if (last < nkt) nkt = last;
  }

  // Register staging of one key/value tile.
  constexpr int K_LOADS = DH * AT_BN * TILE_K / 8 / AT_THREADS;  // 16-byte chunks per lane
  u32x4 rk[K_LOADS];
  u32x4 rv[8];
  const int v_kb = tid & 7;          // key block (8 keys)
  const int v_db = tid >> 3;         // d block (8 d) ; valid when v_db < DM/8
  const bool v_active = v_db < DM / 8;

  auto load_tile = [&](int64_t kt) {
    const int64_t k0 = kt * AT_BN;
    if (KVEC) {
#pragma unroll
      for (int i = 0; i < K_LOADS; ++i) {
        const int e = i * AT_THREADS + tid;
        const int key = e / (DM / 8), dch = e % (DM / 8);
        const int64_t kp = k0 + key;
        rk[i] = kp < g.Sk ? *(const u32x4*)(K + kp * g.ks[2] + dch * 8) : u32x4{0u, 0u, 0u, 0u};
      }
      if (v_active) {
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const int64_t kp = k0 + v_kb * 8 + r;
          rv[r] = kp < g.Sk ? *(const u32x4*)(V + kp * g.vs[2] + v_db * 8) : u32x4{0u, 0u, 0u, 0u};
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < K_LOADS; ++i) {
        const int e = i * AT_THREADS + tid;
        const int key = e / (DM / 8), dch = e % (DM / 8);
        const int64_t kp = k0 + key;
        uint16_t tmp[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int64_t d = dch * 8 + u;
          tmp[u] = (kp < g.Sk && d < g.D) ? K[kp * g.ks[2] + d * g.ks[3]] : (uint16_t)0;
        }
        rk[i] = *(const u32x4*)tmp;
      }
      if (v_active) {
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const int64_t kp = k0 + v_kb * 8 + r;
          uint16_t tmp[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int64_t d = v_db * 8 + u;
            tmp[u] = (kp < g.Sk && d < g.D) ? V[kp * g.vs[2] + d * g.vs[3]] : (uint16_t)0;
          }
          rv[r] = *(const u32x4*)tmp;
        }
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < K_LOADS; ++i) {
      const int e = i * AT_THREADS + tid;
      const int key = e / (DM / 8), dch = e % (DM / 8);
      const int hf = dch >> 3, c = dch & 7;
      *(u32x4*)(sK + hf * AT_BN * TILE_K + key * TILE_K + swz(key, c) * 8) = rk[i];
    }
    if (v_active) {
      u32x4 tv[8];
      transpose8x8(rv, tv);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int d = v_db * 8 + j;
        u32x2* dst = (u32x2*)(sVt + d * VT_STRIDE + v_kb * 8);
        dst[0] = u32x2{tv[j][0], tv[j][1]};
        dst[1] = u32x2{tv[j][2], tv[j][3]};
      }
    }
  };

  if (nkt > 0) {
    load_tile(0);
    store_tile();
  }
  __syncthreads();
  for (int64_t kt = 0; kt < nkt; ++kt) {
    if (kt + 1 < nkt) load_tile(kt + 1);
    const int64_t k0 = kt * AT_BN;
    // S^T = K . Q^T  (two 32-key blocks)
    floatx16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] = 0.f;
#pragma unroll
      for (int dd = 0; dd < DSUB; ++dd) {
        const int hf = dd >> 2;
        const int chunk = (dd & 3) * 2 + half;
        const int row = kb * 32 + (lane & 31);
        const frag ka = *(const frag*)(sK + hf * AT_BN * TILE_K + row * TILE_K + swz(row, chunk) * 8);
        s[kb] = mfma_traits<T>::mma(ka, qf[dd], s[kb]);
      }
    }
    // Masks: keys past the end, and keys after the query when causal.
    const bool need_mask = (k0 + AT_BN > g.Sk) || (g.causal && k0 + AT_BN - 1 > q0 + wave * 32);
    if (need_mask) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t key = k0 + kb * 32 + acc_row(r, lane);
          if (key >= g.Sk || (g.causal && qpos < key)) s[kb][r] = -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_i, mx);
    float lsum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(s[kb][r] - m_new);
        s[kb][r] = p;
        lsum += p;
      }
    lsum += __shfl_xor(lsum, 32, 64);
    const float alpha = __builtin_amdgcn_exp2f(m_i - m_new);
    l_i = l_i * alpha + lsum;
    m_i = m_new;
#pragma unroll
    for (int i = 0; i < DBLK; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) o_acc[i][r] *= alpha;
    // O^T += V^T . P^T over four 16-key slices.
#pragma unroll
    for (int t = 0; t < AT_BN / 16; ++t) {
      uint16_t pt[8];
#pragma unroll
      for (int sl = 0; sl < 8; ++sl) pt[sl] = elem<T>::from_float(s[t >> 1][8 * (t & 1) + sl]);
      const frag pf = __builtin_bit_cast(frag, *(const u32x4*)pt);
#pragma unroll
      for (int i = 0; i < DBLK; ++i) {
        const int d = i * 32 + (lane & 31);
        const uint16_t* rowp = sVt + d * VT_STRIDE;
        const u32x2 lo = *(const u32x2*)(rowp + (2 * t) * 8 + half * 4);
        const u32x2 hi = *(const u32x2*)(rowp + (2 * t + 1) * 8 + half * 4);
        const frag vf = __builtin_bit_cast(frag, u32x4{lo[0], lo[1], hi[0], hi[1]});
        o_acc[i] = mfma_traits<T>::mma(vf, pf, o_acc[i]);
      }
    }
    __syncthreads();
    if (kt + 1 < nkt) {
      store_tile();
      __syncthreads();
    }
  }

  // o = acc / l, staged through LDS per 64-wide slice of d so that each lane then
  // writes 4 consecutive d of one query row (lanes 0-15 cover 64 d of a row).
  {
    const float inv = 1.0f / l_i;
    constexpr int ST = 65;  // padded row: lane-per-row writes hit distinct banks
    float* stage = reinterpret_cast<float*>(smem) + wave * (32 * ST);
    constexpr int PASSES = (DM + 63) / 64;
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        if (ps * 2 + jb < DBLK) {
#pragma unroll
          for (int r = 0; r < 16; ++r)
            stage[(lane & 31) * ST + jb * 32 + acc_row(r, lane)] = o_acc[ps * 2 + jb][r] * inv;
        }
      }
      __syncthreads();
      for (int e = lane; e < 32 * 16; e += 64) {
        const int row = e >> 4, grp = (e & 15) * 4;
        const int64_t qp = q0 + wave * 32 + row;
        const int d0 = ps * 64 + grp;
        if (qp >= g.Sq || d0 >= g.D) continue;
        const float* sp = stage + row * ST + grp;
        const float4 v4 = {sp[0], sp[1], sp[2], sp[3]};
        const int64_t ob = b * g.os[0] + h * g.os[1] + qp * g.os[2];
        if (g.o_dtype != NT_DTYPE_F32 && g.os[3] == 1 && d0 + 4 <= g.D && ((ob + d0) & 3) == 0) {
          uint16_t hv[4];
          const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
          for (int u = 0; u < 4; ++u)
            hv[u] = g.o_dtype == NT_DTYPE_F16 ? float_to_f16_bits(vv[u]) : float_to_bf16_bits(vv[u]);
          *(u32x2*)((uint16_t*)g.o + ob + d0) = *(const u32x2*)hv;
        } else {
          const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
          for (int u = 0; u < 4 && d0 + u < g.D; ++u) store_from_float(g.o, ob + (d0 + u) * g.os[3], g.o_dtype, vv[u]);
        }
      }
      __syncthreads();
    }
  }
}

// Fast path (unit d-stride, 16-byte aligned rows, D == DM, buffer offsets within 32
// bits): the same math as attention_body, eight waves of 32 queries per workgroup (two
// waves per SIMD: one's softmax overlaps the other's matrix work), with
//   - K and V fetched through buffer resources whose range ends at the last key, so
//     keys past Sk read as zeros with no per-load branch, at scalar per-tile offsets;
//     waves 0-3 fetch K, waves 4-7 fetch V and transpose it in 4 (key) x 8 (d) blocks
//     with v_perm_b32;
//   - two LDS stages, so one barrier per key tile: at the top of tile kt every wave has
//     finished tile kt - 1 (whose stage now takes tile kt + 1) and stored tile kt;
//   - lazy rescaling: the running max m is only raised when a tile's max exceeds it by
//     more than RESCALE_LOG2 (then o, l are rescaled), so p = exp2(s - m) stays below
//     2^RESCALE_LOG2 and most tiles skip the rescale; o / l is unchanged mathematically
//     and p keeps the input type's relative precision.  The first tile sets m to its
//     exact max;
//   - the shift by m inside the matrix core: each score accumulator starts at -m;
//   - row sums of the rounded p (the values the product with V uses) on the matrix core,
//     one extra MFMA per 16-key slice against a block of ones;
//   - p rounded two at a time (v_cvt_pk_{f16,bf16}_f32, round to nearest even).
// Its LDS reads (16 KiB of K and 16 KiB of V fragments per wave and key tile) are the
// bound next to the matrix core; halving them needs two query blocks per wave, which
// does not fit two waves per SIMD.
namespace attn {
// V^T rows: 64 keys + 8 pad (144-byte rows: the 16-byte fragment reads of 8 consecutive
// rows fall in 8 distinct 16-byte bank groups).  Within each 16-key slice the keys are
// stored in the order a lane's P^T slots take them, 0-3, 8-11 | 4-7, 12-15, so a V^T
// fragment (keys 16t + (s / 4) * 8 + half * 4 + s % 4, s = 0..7) is 16 contiguous bytes
// at position 16t + 8 half.
constexpr int VT_STRIDE = TILE_K + 8;
// Position of the 4-key group starting at key 4 kq.
__host__ __device__ constexpr int vt_pos(int kq) { return (kq >> 2) * 16 + ((kq & 1) << 3) + ((kq & 2) << 1); }
constexpr float RESCALE_LOG2 = 8.0f;
template <int DM>
struct Geo {
  static constexpr int DH = DM / 64, DSUB = DM / 16, DBLK = DM / 32;
  static constexpr int K_ELEMS = DH * AT_BN * TILE_K;  // K tile [d-half][key][64 d]
  static constexpr int BUF = K_ELEMS + DM * VT_STRIDE;  // + V^T tile [d][64 keys + pad]
  static constexpr int CPR = DM / 8;                    // 16-byte chunks per key row
  static constexpr int K_LOADS = AT_BN * CPR / AT_THREADS;
  static constexpr int KEYS_PER_LOAD = AT_THREADS / CPR;
};
__device__ __forceinline__ uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
  return __builtin_amdgcn_perm(s0, s1, sel);
}
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf162_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));
// Two fp32 values rounded (to nearest even) to the input type, packed low | high << 16.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack2<f16_t>(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_t{lo, hi}, half2_t));
}
template <>
__device__ __forceinline__ uint32_t pack2<bf16_t>(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_t{lo, hi}, bf162_t));
}
// A fragment of eight ones (the a operand that turns an MFMA into column sums).
template <typename T>
__device__ __forceinline__ typename mfma_traits<T>::frag ones_frag() {
  const uint32_t one2 = pack2<T>(1.0f, 1.0f);
  return __builtin_bit_cast(typename mfma_traits<T>::frag, u32x4{one2, one2, one2, one2});
}
}  // namespace attn

template <typename T, int DM, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) void attention_fast_kernel(
    AttnArgs g) {
  constexpr int QB = 1;  // query blocks of 32 per wave
  using G = attn::Geo<DM>;
  typedef typename mfma_traits<T>::frag frag;
  constexpr int WQ = 32 * QB;    // queries per wave (QB blocks of 32)
  constexpr int BM = NW * WQ;    // queries per workgroup
  constexpr int STAGE_ELEMS = NW * 32 * 65 * 2;  // output staging, one block per wave (fp32)
  constexpr int SMEM = 2 * G::BUF > STAGE_ELEMS ? 2 * G::BUF : STAGE_ELEMS;
  __shared__ __attribute__((aligned(16))) uint16_t smem[SMEM];
  char* lds = (char*)smem;

  const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int qb_id;
  int64_t bh;
  block_order(g, blockIdx.x, qb_id, bh);
  const int64_t b = bh / g.H, h = bh % g.H;
  const int q0 = qb_id * BM;
  const int qw = q0 + wave * WQ;  // first query of this wave
  const int Sk = (int)g.Sk;
  const int D = (int)g.D;  // DM / 2 < D <= DM, a multiple of 8
  const uint16_t* Q = (const uint16_t*)g.q + b * g.qs[0] + h * g.qs[1];

  // Q^T fragments of this lane's queries (one per block), pre-scaled and rounded to the
  // input type.  The raw rows are loaded here and scaled only once the first key tile's
  // loads are in flight too, so that the two fetches share one memory latency.
  int qpos[QB];
  frag qf[QB][G::DSUB];
  u32x4 qraw[QB][G::DSUB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    qpos[qb] = qw + qb * 32 + (lane & 31);
#pragma unroll
    for (int dd = 0; dd < G::DSUB; ++dd) {
      qraw[qb][dd] = u32x4{0u, 0u, 0u, 0u};
      if (qpos[qb] < g.Sq && dd * 16 + half * 8 < D)
        qraw[qb][dd] = *(const u32x4*)(Q + (int64_t)qpos[qb] * g.qs[2] + dd * 16 + half * 8);
    }
  }
  auto scale_q = [&]() {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int dd = 0; dd < G::DSUB; ++dd) {
        uint16_t tmp[8];
        const uint16_t* hv = (const uint16_t*)&qraw[qb][dd];
#pragma unroll
        for (int u = 0; u < 8; ++u) tmp[u] = elem<T>::from_float(elem<T>::to_float(hv[u]) * g.q_scale);
        qf[qb][dd] = __builtin_bit_cast(frag, *(const u32x4*)tmp);
      }
  };

  // Tile loaders, 256 lanes per operand: with four waves every lane fetches both K and V;
  // with eight, waves 0-3 fetch K and waves 4-7 fetch V (lane index lt within the 256).
  // K: load i brings key i * KEYS_PER_LOAD + kr, chunk kc.  V: a 4 (key) x 8 (d) block,
  // keys 4 kq .. 4 kq + 3, d 8 db .. 8 db + 7 (lanes with db >= DM / 8 idle when DM = 64).
  const int lt = tid & (AT_THREADS - 1);
  const bool k_role = NW == 4 || wave < 4;
  const bool v_role = (NW == 4 || wave >= 4) && (lt >> 4) < DM / 8;
  const int ks2b = (int)g.ks[2] * 2, vs2b = (int)g.vs[2] * 2;
  // Both resources end at the last key's D-th element.  A head dim D below DM (a multiple
  // of 8) leaves K chunks kc >= D / 8 zero (they meet Q's zero padding in the scores); V's
  // chunks past D reach only output rows d >= D, which are never stored.
  const __amdgpu_buffer_rsrc_t rsK = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint16_t*)g.k + b * g.ks[0] + h * g.ks[1]), (short)0, (Sk - 1) * ks2b + D * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsV = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint16_t*)g.v + b * g.vs[0] + h * g.vs[1]), (short)0, (Sk - 1) * vs2b + D * 2, 0x00020000);
  const int kr = lt / G::CPR, kc = lt % G::CPR;
  const bool k_ok = kc * 8 < D;
  const int vK = kr * ks2b + kc * 16;
  int k_st[G::K_LOADS];
#pragma unroll
  for (int i = 0; i < G::K_LOADS; ++i) {
    const int key = i * G::KEYS_PER_LOAD + kr;
    k_st[i] = ((kc >> 3) * AT_BN * TILE_K + key * TILE_K + swz(key, kc & 7) * 8) * 2;
  }
  const int kq = lt & 15, db = lt >> 4;
  const int vV = kq * 4 * vs2b + db * 16;
  const int v_st = (G::K_ELEMS + db * 8 * attn::VT_STRIDE + attn::vt_pos(kq)) * 2;

  constexpr int RK = NW == 4 ? G::K_LOADS : 0;  // K registers beside the shared ones
  u32x4 rl[4 > G::K_LOADS ? 4 : G::K_LOADS];    // V rows (and K chunks with eight waves)
  u32x4 rk_own[RK > 0 ? RK : 1];
  u32x4* rk = NW == 4 ? rk_own : rl;
  auto load_tile = [&](int kt) {
    const int k0 = kt * AT_BN;
    if (k_role) {
#pragma unroll
      for (int i = 0; i < G::K_LOADS; ++i)
        rk[i] = k_ok ? __builtin_amdgcn_raw_buffer_load_b128(rsK, vK, (k0 + i * G::KEYS_PER_LOAD) * ks2b, 0)
                     : u32x4{0u, 0u, 0u, 0u};
    }
    if (v_role) {
#pragma unroll
      for (int r = 0; r < 4; ++r) rl[r] = __builtin_amdgcn_raw_buffer_load_b128(rsV, vV, (k0 + r) * vs2b, 0);
    }
  };
  auto store_tile = [&](int buf) {
    char* base = lds + buf * (G::BUF * 2);
    if (k_role) {
#pragma unroll
      for (int i = 0; i < G::K_LOADS; ++i) *(u32x4*)(base + k_st[i]) = rk[i];
    }
    if (v_role) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int d = j >> 1;
        const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
        *(u32x2*)(base + v_st + j * attn::VT_STRIDE * 2) =
            u32x2{attn::perm(rl[1][d], rl[0][d], sel), attn::perm(rl[3][d], rl[2][d], sel)};
      }
    }
  };

  floatx16 o_acc[QB][G::DBLK];
  // m_i: the running max, kept lazily; negm: -m_i in every register, the starting value of
  // each score accumulator (zero for the first tile, whose max sets m_i exactly); l_acc:
  // row sums of the rounded p, accumulated by the matrix core against a block of ones
  // (every register of a lane holds its query's sum).
  float m_i[QB];
  floatx16 negm[QB], l_acc[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_i[qb] = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      negm[qb][r] = 0.f;
      l_acc[qb][r] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < G::DBLK; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) o_acc[qb][i][r] = 0.f;
  }
  const frag ones = attn::ones_frag<T>();

  int nkt = (Sk + AT_BN - 1) / AT_BN;
  if (g.causal) nkt = min(nkt, (q0 + BM - 1) / AT_BN + 1);

  if (nkt > 0) load_tile(0);
  scale_q();
  if (nkt > 0) {
    store_tile(0);
    if (nkt > 1) load_tile(1);
  }
  // Causal: tiles whose first key follows every query of this wave would only add masked
  // scores (p = 0), so the wave computes up to its own last tile nkt_w and then only takes
  // its part in the workgroup's loads and barriers (a separate loop, so the main one
  // carries no branch around its body).
  const int nkt_w = g.causal ? min(nkt, (qw + WQ - 1) / AT_BN + 1) : nkt;
  int kt = 0;
  for (; kt < nkt_w; ++kt) {
    __syncthreads();
    if (kt + 1 < nkt) {
      store_tile((kt + 1) & 1);
      if (kt + 2 < nkt) load_tile(kt + 2);
    }
    const int k0 = kt * AT_BN;
    const uint16_t* sK = smem + (kt & 1) * G::BUF;
    const uint16_t* sVt = sK + G::K_ELEMS;
    // S^T = K . Q^T: per query block two 32-key accumulator chains; each K fragment (read
    // a slice ahead) feeds every query block.
    floatx16 s[QB][2];
    auto k_frag = [&](int kb, int dd) {
      const int hf = dd >> 2;
      const int chunk = (dd & 3) * 2 + half;
      const int row = kb * 32 + (lane & 31);
      return *(const frag*)(sK + hf * AT_BN * TILE_K + row * TILE_K + swz(row, chunk) * 8);
    };
    frag ka[2][2];
    ka[0][0] = k_frag(0, 0);
    ka[0][1] = k_frag(1, 0);
#pragma unroll
    for (int dd = 0; dd < G::DSUB; ++dd) {
      if (dd + 1 < G::DSUB) {
        ka[(dd + 1) & 1][0] = k_frag(0, dd + 1);
        ka[(dd + 1) & 1][1] = k_frag(1, dd + 1);
      }
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
          s[qb][kb] = mfma_traits<T>::mma(ka[dd & 1][kb], qf[qb][dd], dd == 0 ? negm[qb] : s[qb][kb]);
    }
    // Masks: keys past the end, and keys after the query when causal.
    if (k0 + AT_BN > Sk || (g.causal && k0 + AT_BN - 1 > qw)) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = k0 + kb * 32 + acc_row(r, lane);
            if (key >= Sk || (g.causal && qpos[qb] < key)) s[qb][kb][r] = -INFINITY;
          }
    }
    // The scores are already shifted by m_i.  The first tile sets m_i to its max; later
    // tiles raise it where their max passes RESCALE_LOG2 (rescaling o and l to match).
    float delta[QB];
    bool any_grow = false;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[qb][kb][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const bool grow = kt == 0 || mx > attn::RESCALE_LOG2;
      delta[qb] = grow ? mx : 0.f;
      any_grow |= grow;
    }
    if (__builtin_amdgcn_ballot_w64(any_grow)) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        if (kt > 0) {
          const float alpha = __builtin_amdgcn_exp2f(-delta[qb]);
#pragma unroll
          for (int r = 0; r < 16; ++r) l_acc[qb][r] *= alpha;
#pragma unroll
          for (int i = 0; i < G::DBLK; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) o_acc[qb][i][r] *= alpha;
        }
        m_i[qb] += delta[qb];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) s[qb][kb][r] -= delta[qb];
#pragma unroll
        for (int r = 0; r < 16; ++r) negm[qb][r] = -m_i[qb];
      }
    }
    // P^T in the input type (two values per v_cvt_pk).
    frag pf[QB][AT_BN / 16];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int t = 0; t < AT_BN / 16; ++t) {
        u32x4 w;
#pragma unroll
        for (int sl = 0; sl < 4; ++sl) {
          const int r0 = 8 * (t & 1) + 2 * sl;
          w[sl] = attn::pack2<T>(__builtin_amdgcn_exp2f(s[qb][t >> 1][r0]),
                                 __builtin_amdgcn_exp2f(s[qb][t >> 1][r0 + 1]));
        }
        pf[qb][t] = __builtin_bit_cast(frag, w);
      }
    // O^T += V^T . P^T over four 16-key slices; each V^T fragment feeds every query block.
#pragma unroll
    for (int t = 0; t < AT_BN / 16; ++t) {
#pragma unroll
      for (int i = 0; i < G::DBLK; ++i) {
        const int d = i * 32 + (lane & 31);
        const frag vf = *(const frag*)(sVt + d * attn::VT_STRIDE + t * 16 + half * 8);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) o_acc[qb][i] = mfma_traits<T>::mma(vf, pf[qb][t], o_acc[qb][i]);
      }
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) l_acc[qb] = mfma_traits<T>::mma(ones, pf[qb][t], l_acc[qb]);
    }
  }
  for (; kt < nkt; ++kt) {
    __syncthreads();
    if (kt + 1 < nkt) {
      store_tile((kt + 1) & 1);
      if (kt + 2 < nkt) load_tile(kt + 2);
    }
  }
  __syncthreads();  // the output staging below reuses the K/V stages

  // o = acc / l, staged through LDS per 64-wide slice of d so that each lane then
  // writes 4 consecutive d of one query row (lanes 0-15 cover 64 d of a row).
  constexpr int ST = 65;
  float* stage = reinterpret_cast<float*>(smem) + wave * (32 * ST);
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float inv = 1.0f / l_acc[qb][0];
#pragma unroll
    for (int ps = 0; ps < DM / 64; ++ps) {
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          stage[(lane & 31) * ST + jb * 32 + acc_row(r, lane)] = o_acc[qb][ps * 2 + jb][r] * inv;
      wave_lds_order();  // a wave reads back only its own staging rows
#pragma unroll
      for (int e0 = 0; e0 < 32 * 16; e0 += 64) {
        const int e = e0 + lane;
        const int row = e >> 4, grp = (e & 15) * 4;
        const int qp = qw + qb * 32 + row;
        if (qp < g.Sq && ps * 64 + grp < D) {
          const float* sp = stage + row * ST + grp;
          const int64_t ob = b * g.os[0] + h * g.os[1] + (int64_t)qp * g.os[2];
          const int d0 = ps * 64 + grp;
          if (g.o_dtype == elem<T>::code && g.os[3] == 1 && ((ob + d0) & 3) == 0) {
            *(u32x2*)((uint16_t*)g.o + ob + d0) = u32x2{attn::pack2<T>(sp[0], sp[1]), attn::pack2<T>(sp[2], sp[3])};
          } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) store_from_float(g.o, ob + (d0 + u) * g.os[3], g.o_dtype, sp[u]);
          }
        }
      }
      wave_lds_order();  // the next slice rewrites the staging rows after these reads
    }
  }
}

// Pipelined kernel (head dim 128, 16-bit, the fast path's conditions; configuration 1, a
// tuning candidate: on MI355X it runs 5-12 % slower than attention_fast_kernel at the
// B=4, H=32, S=4096 shape, because one wave alone on a SIMD cannot issue the softmax's
// VALU work fast enough beside its MFMAs).  Four waves per workgroup, one per SIMD, each
// owning 64 queries (two blocks of 32), so every K and V^T fragment read from LDS feeds two
// MFMAs and the LDS reads per MFMA halve against the eight-wave kernel.  A wave alone on
// its SIMD has 512 registers (the O^T accumulators and Q live in AGPRs) and overlaps its
// own softmax with its matrix work: iteration j issues
//   phase A: S^T_{j+1} = K_{j+1} . Q^T (16 MFMAs)  beside  P_j = exp2(S_j), row sums
//   phase B: O^T += V_j^T . P_j^T   (16 MFMAs)     beside  the max of S_{j+1} (mask, lazy
//                                                          rescale check)
// so the VALU work of one key tile runs under the MFMAs of the next.  Key tiles of 32,
// in pairs, come from HBM straight into a four-stage LDS ring (one stage per pair, K and V
// in separate halves of LDS) by DMA (buffer_load ... lds), two pairs ahead, one barrier per
// pair:
//   K tile  [key][128 d], 256-byte rows whose 16-byte chunks are XOR-swizzled by key % 16:
//           the S^T operand (32 keys x 8 d per lane) is one ds_read_b128;
//   V tile  [key][128 d] as in HBM, 64-byte chunks XOR-swizzled by key % 4: the O^T
//           operand V^T (32 d x 8 keys per lane) is two ds_read_b64_tr_b16, each giving
//           a lane 4 consecutive keys of its d (lane 4 r + q of a 16-lane group reads key
//           k0 + r at d0 + 4 q .. + 3; lane j receives d0 + j at keys k0 .. k0 + 3).
// The key order inside a 16-key slice is the one of P^T's register slots (slot s of lane
// half h is key 8 (s / 4) + 4 h + s % 4), as in the other kernels.  Row sums of the rounded
// p on the VALU with v_dot2 (two products by one per instruction, fp32 accumulation).
// Math, lazy rescaling and rounding points are those of attention_fast_kernel.
namespace ap {
constexpr int NW = 4;               // waves per workgroup (one per SIMD)
constexpr int WQ = 64;              // queries per wave: two blocks of 32
constexpr int BM = NW * WQ;         // queries per workgroup
constexpr int BN = 32;              // keys per tile (the unit of the math)
constexpr int ROW = 256;            // bytes per key row (128 d)
constexpr int KV = BN * ROW;        // one K or V tile: 8 KiB
constexpr int STAGE = 2 * KV;       // a stage holds a pair of tiles (64 keys) of K, or of V
constexpr int STAGES = 4;
constexpr int VREG = STAGES * STAGE;       // V stages follow the K stages
constexpr int LDS_BYTES = 2 * VREG;        // 128 KiB
typedef short v4i16 __attribute__((ext_vector_type(4)));
// 16 bytes per lane from buffer `rs` at voffset + soffset into LDS at lds_addr + 16 * lane.
__device__ __forceinline__ void load_lds16(u32x4 rs, uint32_t lds_addr, int voffset, int soffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voffset), "s"(rs),
                 "s"(__builtin_amdgcn_readfirstlane(soffset))
               : "memory", "m0");
}
// Buffer resource (uniform: every word read from the first lane, so it lives in SGPRs).
__device__ __forceinline__ u32x4 rsrc(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)base;
  return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)p),
               (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(p >> 32) & 0xffffu),
               (uint32_t)__builtin_amdgcn_readfirstlane(bytes), 0x00020000u};
}
// Row sum of two rounded p values packed in w, accumulated in fp32.
template <typename T>
__device__ __forceinline__ float dot_ones(uint32_t w, float acc);
// Volatile inline assembly so that the compiler keeps each at its place in the schedule
// (as a plain builtin it would sink the row sums past the rescale branch, out of the
// matrix work they are meant to overlap).
template <>
__device__ __forceinline__ float dot_ones<f16_t>(uint32_t w, float acc) {
  asm volatile("v_dot2c_f32_f16 %0, %1, %2" : "+v"(acc) : "v"(w), "v"(0x3c003c00u));
  return acc;
}
template <>
__device__ __forceinline__ float dot_ones<bf16_t>(uint32_t w, float acc) {
  asm volatile("v_dot2c_f32_bf16 %0, %1, %2" : "+v"(acc) : "v"(w), "v"(0x3f803f80u));
  return acc;
}
// x of lane l ^ 32 (v_permlane32_swap on two copies of x: afterwards the first holds the
// low half's values in both halves and the second the high half's).  Inline assembly: the
// builtin with equal operands has been folded to a wrong result.  s_nop 1: the VALU write
// of an operand needs wait states before v_permlane32_swap reads it.
__device__ __forceinline__ void halves(float x, float& lo, float& hi) {
  lo = x;
  hi = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(lo), "+v"(hi));
}
__device__ __forceinline__ float max_halves(float x) {
  float lo, hi;
  halves(x, lo, hi);
  return fmaxf(lo, hi);
}
__device__ __forceinline__ float sum_halves(float x) {
  float lo, hi;
  halves(x, lo, hi);
  return lo + hi;
}
// O^T += V^T . P^T with the accumulator in AGPRs (the scores stay in VGPRs).  Written as
// inline assembly, so the compiler neither sees it as an MFMA nor inserts its wait
// states: the callers do (nop_after_valu before the first of a group whose operands the
// VALU just wrote, nop_after_mfma before the VALU reads an accumulator).
template <typename T>
__device__ __forceinline__ void pv_mma(floatx16& acc, typename mfma_traits<T>::frag a, typename mfma_traits<T>::frag b);
template <>
__device__ __forceinline__ void pv_mma<f16_t>(floatx16& acc, half8 a, half8 b) {
  asm("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
template <>
__device__ __forceinline__ void pv_mma<bf16_t>(floatx16& acc, bf16x8 a, bf16x8 b) {
  asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// Moves of an accumulator between AGPRs and VGPRs, as inline assembly so that every
// definition of an O^T accumulator is an AGPR one (otherwise the register allocator may
// give the loop-carried accumulators VGPRs and copy them around every iteration).
__device__ __forceinline__ floatx16 to_agpr(floatx16 v) {
  floatx16 r;
  asm volatile("" : "=a"(r) : "0"(v));
  return r;
}
template <typename F>
__device__ __forceinline__ F frag_to_agpr(F v) {
  F r;
  asm volatile("" : "=a"(r) : "0"(v));
  return r;
}
__device__ __forceinline__ floatx16 from_agpr(floatx16 a) {
  floatx16 r;
  asm volatile("" : "=v"(r) : "0"(a));
  return r;
}
// Wait states: a VALU write read by an MFMA needs 2; an 8-pass MFMA's result read by the
// VALU (or v_accvgpr_read) needs 11.  Both with margin.
__device__ __forceinline__ void nop_after_valu() { asm volatile("s_nop 4"); }
__device__ __forceinline__ void nop_after_mfma() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 4"); }
// Scheduling group masks of __builtin_amdgcn_sched_group_barrier.
constexpr int SG_VALU = 0x0002 | 0x0400, SG_MFMA = 0x0008, SG_DSR = 0x0100;
}  // namespace ap

template <typename T>
__global__ __launch_bounds__(ap::NW * 64) __attribute__((amdgpu_waves_per_eu(1, 1))) void attention_pipe_kernel(
    AttnArgs g) {
  typedef typename mfma_traits<T>::frag frag;
  __shared__ __attribute__((aligned(1024))) char lds[ap::LDS_BYTES];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;
  const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int qb_id;
  int64_t bh;
  block_order(g, blockIdx.x, qb_id, bh);
  const int b = (int)(bh / g.H), h = (int)(bh % g.H);
  const int q0 = qb_id * ap::BM;
  const int qw = q0 + wave * ap::WQ;  // first query of this wave
  const int Sk = (int)g.Sk, Sq = (int)g.Sq;
  const bool causal = g.causal != 0;

  // Tiles: the workgroup's (up to its last wave's last visible key when causal) and this
  // wave's own (the others only take part in loads and barriers).
  int nkt = (Sk + ap::BN - 1) / ap::BN;
  if (causal) nkt = min(nkt, (q0 + ap::BM - 1) / ap::BN + 1);
  const int nkt_w = causal ? min(nkt, (qw + ap::WQ - 1) / ap::BN + 1) : nkt;
  // First tile holding a key past Sk or, causal, past one of this wave's queries.
  const int first_mask = causal ? min(qw / ap::BN, Sk / ap::BN) : Sk / ap::BN;

  // DMA, per pair of tiles (64 keys, one stage of K and one of V): wave w brings chunks
  // 4 w .. 4 w + 3 (1 KiB each: keys 4 i .. 4 i + 3) of both.
  const int ks2b = (int)g.ks[2] * 2, vs2b = (int)g.vs[2] * 2;
  const u32x4 rsK =
      ap::rsrc((const uint16_t*)g.k + b * g.ks[0] + h * g.ks[1], (uint32_t)((Sk - 1) * ks2b + ap::ROW));
  const u32x4 rsV =
      ap::rsrc((const uint16_t*)g.v + b * g.vs[0] + h * g.vs[1], (uint32_t)((Sk - 1) * vs2b + ap::ROW));
  int vk[4], vv[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int key = 4 * (4 * wave + u) + (lane >> 4), p = lane & 15;
    vk[u] = key * ks2b + (p ^ (key & 15)) * 16;
    vv[u] = key * vs2b + ((((p >> 2) ^ (key & 3)) << 2) | (p & 3)) * 16;
  }
  const int kstep = 2 * ap::BN * ks2b, vstep = 2 * ap::BN * vs2b;
  const int npair = (nkt + 1) / 2;  // tile pairs of the workgroup
  auto issue = [&](int tp) {        // tile pair tp into stage tp % 4
    const uint32_t st = lds0 + (uint32_t)((tp & 3) * ap::STAGE) + (uint32_t)(4 * wave * 1024);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      ap::load_lds16(rsK, st + u * 1024, vk[u], tp * kstep);
      ap::load_lds16(rsV, st + ap::VREG + u * 1024, vv[u], tp * vstep);
    }
  };
  issue(0);
  if (npair > 1) issue(1);
  if (npair > 2) issue(2);

  // Q^T fragments of this lane's two queries, pre-scaled and rounded to the input type.
  frag qf[2][8];
  int qpos[2];
  {
    const uint16_t* Q = (const uint16_t*)g.q + b * g.qs[0] + h * g.qs[1];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      qpos[qb] = qw + qb * 32 + (lane & 31);
#pragma unroll
      for (int dd = 0; dd < 8; ++dd) {
        u32x4 raw = {0u, 0u, 0u, 0u};
        if (qpos[qb] < Sq) raw = *(const u32x4*)(Q + (int64_t)qpos[qb] * g.qs[2] + dd * 16 + half * 8);
        uint16_t tmp[8];
        const uint16_t* hv = (const uint16_t*)&raw;
#pragma unroll
        for (int u = 0; u < 8; ++u) tmp[u] = elem<T>::from_float(elem<T>::to_float(hv[u]) * g.q_scale);
        qf[qb][dd] = ap::frag_to_agpr(__builtin_bit_cast(frag, *(const u32x4*)tmp));  // MFMA b operands from AGPRs
      }
    }
  }
  // Output addressing, computed now so the key loop carries no 64-bit arguments.
  uint16_t* const obase = (uint16_t*)g.o + (int64_t)b * g.os[0] + (int64_t)h * g.os[1];
  const int64_t os2 = g.os[2], os3 = g.os[3];
  const int o_dtype = g.o_dtype;

  // LDS read addresses (bytes, stage 0).  K fragment dd: key lane % 32, chunk 2 dd + half.
  // V^T fragment of d block i: lane (group gq, r, q) at key 4 (gq / 2) + r (+ 16 t + 8 R),
  // d 32 i + 16 (gq % 2) + 4 q; key % 4 = r picks the 64-byte chunk i ^ r.
  int k_rd[8], v_rd[4];
#pragma unroll
  for (int dd = 0; dd < 8; ++dd) k_rd[dd] = (lane & 31) * ap::ROW + (((2 * dd + half) ^ (lane & 15)) * 16);
  {
    const int gq = lane >> 4, r = (lane & 15) >> 2, q = lane & 3;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      v_rd[i] = ap::VREG + (4 * (gq >> 1) + r) * ap::ROW + ((i ^ r) * 64) + (16 * (gq & 1) + 4 * q) * 2;
  }

  floatx16 o[2][4];  // O^T accumulators, in AGPRs
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int i = 0; i < 4; ++i) o[qb][i] = ap::to_agpr(floatx16{});
  floatx16 s[2][2];  // [buffer][query block]: S^T of a tile, shifted by -m
  floatx16 negm[2];  // -m in every register: the first MFMA's accumulator input
  float m[2], ls[2];
  u32x4 pw[2][2];  // [query block][16-key slice]: P^T, two rounded values per word

  // Masking through the accumulator's starting value: for a tile that holds a key past Sk
  // or (causal) past one of this wave's queries, the first MFMA of its scores starts from
  // -inf at those positions (base elsewhere), so the scores come out masked.
  auto masked_start = [&](floatx16 (&c)[2], const float (&base)[2], int k0) {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int lim = (causal ? min(qpos[qb] + 1, Sk) : Sk) - k0 - half * 4;  // keys below lim stay
#pragma unroll
      for (int r = 0; r < 16; ++r) c[qb][r] = (r >> 2) * 8 + (r & 3) < lim ? base[qb] : -INFINITY;
    }
  };
  // Top of an odd iteration j = 2 tp - 1: tile pair tp (tiles j + 1, j + 2) landed (own
  // loads, then everyone's: the barrier), and every wave is done with pair tp - 2, whose
  // stage takes pair tp + 2.
  auto sync_pair = [&](int tp) {
    if (tp + 1 < npair)
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("s_barrier" ::: "memory");
    if (tp + 2 < npair) issue(tp + 2);
  };
  // Stage moves of the fragment read addresses (to the stage of pair tp from tp - 1).
  auto stage_delta = [](int tp) { return ((tp & 3) - ((tp - 1) & 3)) * ap::STAGE; };

  // Tile 0: scores, exact max.
  if (npair > 2)
    asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
  else if (npair > 1)
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  asm volatile("s_barrier" ::: "memory");
  {
    floatx16 start[2] = {};
    if (first_mask == 0) masked_start(start, {0.f, 0.f}, 0);
#pragma unroll
    for (int dd = 0; dd < 8; ++dd) {
      const frag kf = *(const frag*)(lds + k_rd[dd]);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) s[0][qb] = mfma_traits<T>::mma(kf, qf[qb][dd], dd == 0 ? start[qb] : s[0][qb]);
    }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      float mx = s[0][qb][0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[0][qb][r]);
      mx = ap::max_halves(mx);
      m[qb] = mx;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[0][qb][r] -= mx;
        negm[qb][r] = -mx;
      }
      ls[qb] = 0.f;
    }
  }

  // P^T item w (0..15): the pair of rounded p in word sl of slice t of query block qb,
  // from the scores of buffer B.
  auto p_item = [&](auto b_c, auto w_c) {
    constexpr int B = decltype(b_c)::value, W = decltype(w_c)::value;
    // items 0-3: query block 0, slice 0; 4-7: block 1, slice 0; 8-11: block 0, slice 1; 12-15: block 1, slice 1
    constexpr int QB = (W >> 2) & 1, TT = W >> 3, SL = W & 3;
    constexpr int r0 = 8 * TT + 2 * SL;
    pw[QB][TT][SL] = attn::pack2<T>(__builtin_amdgcn_exp2f(s[B][QB][r0]), __builtin_amdgcn_exp2f(s[B][QB][r0 + 1]));
  };
  auto sum_item = [&](auto w_c) {
    constexpr int W = decltype(w_c)::value;
    constexpr int QB = (W >> 2) & 1, TT = W >> 3, SL = W & 3;
    ls[QB] = ap::dot_ones<T>(pw[QB][TT][SL], ls[QB]);
  };

  // Iteration j (P = j % 2; S_j in buffer P).  Tile t lives in stage (t / 2) % 4 at
  // KV * (t % 2); k_rd points at the stage of K_{j+1}, v_rd at that of V_j.  The last
  // iteration of a wave (no tile j + 1) computes scores from whatever the stage holds and
  // leaves them unused: its max takes no part in the rescale check, nothing reads them.
  auto iter = [&](auto p_c, int j) {
    constexpr int P = decltype(p_c)::value;
    constexpr int CUR = P, NXT = P ^ 1;
    constexpr int OFF_K1 = P == 0 ? ap::KV : 0, OFF_V = P == 0 ? 0 : ap::KV;
    const bool has_next = j + 1 < nkt_w;
    if constexpr (P == 1) {
      const int tp = (j + 1) / 2;
      sync_pair(tp);
      const int dlt = stage_delta(tp);
#pragma unroll
      for (int dd = 0; dd < 8; ++dd) k_rd[dd] += dlt;
    } else if (j > 0) {
      const int dlt = stage_delta(j / 2);
#pragma unroll
      for (int i = 0; i < 4; ++i) v_rd[i] += dlt;
    }
    // Tiles from first_mask on are the last of the wave: negm takes -inf at their masked
    // positions from here on (a rescale resets it, and the next iteration sets it again).
    if (j + 1 >= first_mask && has_next) masked_start(negm, {-m[0], -m[1]}, (j + 1) * ap::BN);
    __builtin_amdgcn_sched_barrier(0);
    // Phase A: all eight K fragments of tile j + 1 read at once, then eight groups of two
    // MFMAs of S_{j+1}, with P^T items 0..11 of tile j spread over them (1.5 per group)
    // and one V^T fragment of tile j read per group for phase B.
    auto v_frag = [&](int t, int i) {
      const char* p = lds + v_rd[i] + OFF_V + t * 16 * ap::ROW;
      const ap::v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) ap::v4i16*)p);
      const ap::v4i16 hi =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) ap::v4i16*)(p + 8 * ap::ROW));
      const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
      return __builtin_bit_cast(frag, u32x4{l2[0], l2[1], h2[0], h2[1]});
    };
    frag kf[8], vf[8];
#pragma unroll
    for (int dd = 0; dd < 8; ++dd) kf[dd] = *(const frag*)(lds + k_rd[dd] + OFF_K1);
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, 8>([&](auto dd_c) {
      constexpr int DD = decltype(dd_c)::value;
      static_for<0, 12>([&](auto w_c) {
        constexpr int W = decltype(w_c)::value;
        if constexpr (W * 2 / 3 == DD && W % 3 == 0) p_item(std::integral_constant<int, CUR>{}, w_c);
      });
      s[NXT][0] = mfma_traits<T>::mma(kf[DD], qf[0][DD], DD == 0 ? negm[0] : s[NXT][0]);
      vf[DD] = v_frag(DD >> 2, DD & 3);
      static_for<0, 12>([&](auto w_c) {
        constexpr int W = decltype(w_c)::value;
        if constexpr (W * 2 / 3 == DD && W % 3 != 0) p_item(std::integral_constant<int, CUR>{}, w_c);
      });
      s[NXT][1] = mfma_traits<T>::mma(kf[DD], qf[1][DD], DD == 0 ? negm[1] : s[NXT][1]);
      __builtin_amdgcn_sched_barrier(0);
    });
    __builtin_amdgcn_sched_barrier(0);
    // Phase B: eight groups (slice t, d block i) of two MFMAs of O^T += V_j^T . P_j^T; P^T
    // items 12..15 in groups 0..3, the row sums and the max of S_{j+1} in the rest.
    float mx[2] = {-INFINITY, -INFINITY};
    static_for<0, 8>([&](auto g_c) {
      constexpr int G = decltype(g_c)::value, t = G >> 2, i = G & 3;
      if constexpr (G == 0) ap::nop_after_valu();
      ap::pv_mma<T>(o[0][i], vf[G], __builtin_bit_cast(frag, pw[0][t]));
      if constexpr (G < 4) p_item(std::integral_constant<int, CUR>{}, std::integral_constant<int, 12 + G>{});
      if constexpr (G >= 4) {
        constexpr int R = 4 * (G - 4);
        mx[0] = fmaxf(fmaxf(mx[0], s[NXT][0][R]), s[NXT][0][R + 1]);
        mx[0] = fmaxf(fmaxf(mx[0], s[NXT][0][R + 2]), s[NXT][0][R + 3]);
      }
      if constexpr (G == 3) ap::nop_after_valu();
      ap::pv_mma<T>(o[1][i], vf[G], __builtin_bit_cast(frag, pw[1][t]));
      if constexpr (G >= 4) {
        constexpr int R = 4 * (G - 4);
        mx[1] = fmaxf(fmaxf(mx[1], s[NXT][1][R]), s[NXT][1][R + 1]);
        mx[1] = fmaxf(fmaxf(mx[1], s[NXT][1][R + 2]), s[NXT][1][R + 3]);
        static_for<0, 4>([&](auto u_c) { sum_item(std::integral_constant<int, 4 * (G - 4) + decltype(u_c)::value>{}); });
      }
      __builtin_amdgcn_sched_barrier(0);
    });
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) mx[qb] = ap::max_halves(mx[qb]);
    // Lazy rescale: raise m only where tile j + 1's max passes it by RESCALE_LOG2.
    const bool grow0 = has_next && mx[0] > attn::RESCALE_LOG2, grow1 = has_next && mx[1] > attn::RESCALE_LOG2;
    if (__builtin_amdgcn_ballot_w64(grow0 || grow1)) {
      ap::nop_after_mfma();
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const float delta = (qb == 0 ? grow0 : grow1) ? mx[qb] : 0.f;
        const float alpha = __builtin_amdgcn_exp2f(-delta);
        ls[qb] *= alpha;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[qb][i] = ap::to_agpr(ap::from_agpr(o[qb][i]) * alpha);
        m[qb] += delta;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          s[NXT][qb][r] -= delta;
          negm[qb][r] = -m[qb];
        }
      }
    }
  };
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  for (int j = 0;; j += 2) {
    iter(P0{}, j);
    if (j + 1 >= nkt_w) break;
    iter(P1{}, j + 1);
    if (j + 2 >= nkt_w) break;
  }
  // Tiles of later waves (causal): loads and barriers only.
  for (int jj = nkt_w; jj < nkt; ++jj)
    if (jj & 1) sync_pair((jj + 1) / 2);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  asm volatile("s_barrier" ::: "memory");  // the output staging reuses the stages
  ap::nop_after_mfma();

  // o = acc / l, staged per wave through LDS 64 d at a time; each lane then writes 4
  // consecutive d of one query row.
  constexpr int STR = 65;
  float* stage = reinterpret_cast<float*>(lds) + wave * (32 * STR);
  const bool ovec = o_dtype == elem<T>::code && os3 == 1;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const float inv = 1.0f / ap::sum_halves(ls[qb]);
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
      wave_lds_order();
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        const floatx16 ov = ap::from_agpr(o[qb][ps * 2 + jb]);
#pragma unroll
        for (int r = 0; r < 16; ++r) stage[(lane & 31) * STR + jb * 32 + acc_row(r, lane)] = ov[r] * inv;
      }
      wave_lds_order();
#pragma unroll
      for (int e0 = 0; e0 < 32 * 16; e0 += 64) {
        const int e = e0 + lane;
        const int row = e >> 4, grp = (e & 15) * 4;
        const int qp = qw + qb * 32 + row;
        if (qp < Sq) {
          const float* sp = stage + row * STR + grp;
          const int64_t ob = (int64_t)qp * os2;
          const int d0 = ps * 64 + grp;
          if (ovec && (((uintptr_t)(obase + ob + d0)) & 7) == 0) {
            *(u32x2*)(obase + ob + d0) = u32x2{attn::pack2<T>(sp[0], sp[1]), attn::pack2<T>(sp[2], sp[3])};
          } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) store_from_float(obase, ob + (d0 + u) * os3, o_dtype, sp[u]);
          }
        }
      }
    }
  }
}

// Vector-load variant: two waves per SIMD (two workgroups per CU) so that one
// workgroup's softmax and LDS traffic overlap the other's matrix work.
template <typename T, int DM>
__global__ __launch_bounds__(AT_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void attention_kernel(AttnArgs g) {
  attention_body<T, DM, true>(g);
}

// Element-wise loads for unusual strides or head dims.
template <typename T, int DM>
__global__ __launch_bounds__(AT_THREADS) void attention_generic_kernel(AttnArgs g) {
  attention_body<T, DM, false>(g);
}

// config: 0 = attention_fast_kernel where its conditions hold, else the four-wave kernels;
// 1 = attention_pipe_kernel (head dim 128, the fast conditions); 2 = attention_fast_kernel
// (the fast conditions); 3 = the four-wave kernels (attention_kernel, or
// attention_generic_kernel for other strides).
// A forced configuration whose conditions do not hold returns NT_ERR_INVALID unlaunched.
// No keys: every query's weights are an empty softmax and its output is zero (as torch's
// scaled_dot_product_attention defines it); o is filled, element by element over its strides.
__global__ __launch_bounds__(256) void attention_empty_keys_kernel(void* o, AttnArgs g) {
  const int64_t total = g.B * g.H * g.Sq * g.D;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int64_t d = e % g.D, t = e / g.D;
    const int64_t s = t % g.Sq, u = t / g.Sq;
    const int64_t h = u % g.H, b = u / g.H;
    store_from_float(o, b * g.os[0] + h * g.os[1] + s * g.os[2] + d * g.os[3], g.o_dtype, 0.f);
  }
}

static int attention_empty_keys(void* o, const int64_t* os, int o_dtype, int64_t B, int64_t H, int64_t Sq, int64_t D,
                                hipStream_t stream) {
  AttnArgs g{};
  g.B = B; g.H = H; g.Sq = Sq; g.D = D; g.o_dtype = o_dtype;
  for (int i = 0; i < 4; ++i) g.os[i] = os[i];
  const int64_t blocks = std::min<int64_t>(cdiv(B * H * Sq * D, 256), 4096);
  hipLaunchKernelGGL(attention_empty_keys_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, o, g);
  return launch_status();
}

template <typename T>
static int attention_launch(const void* q, const int64_t* qs, const void* k, const int64_t* ks, const void* v,
                            const int64_t* vs, void* o, const int64_t* os, int o_dtype, int64_t B, int64_t H,
                            int64_t Sq, int64_t Sk, int64_t D, float q_scale, int causal, hipStream_t stream,
                            int config = 0) {
  if (config < 0 || config > 3) return NT_ERR_INVALID;
  if (B < 0 || H < 0 || Sq < 0 || Sk < 0 || D < 0 || D > 128) return NT_ERR_INVALID;
  if (!valid_dtype(o_dtype)) return NT_ERR_INVALID;
  if (B * H * Sq * D == 0) return 0;
  if (!o || !os) return NT_ERR_INVALID;
  if (Sk == 0) return attention_empty_keys(o, os, o_dtype, B, H, Sq, D, stream);
  if (!q || !k || !v || !qs || !ks || !vs) return NT_ERR_INVALID;
  AttnArgs g{};
  g.q = q; g.k = k; g.v = v; g.o = o;
  for (int i = 0; i < 4; ++i) {
    g.qs[i] = qs[i];
    g.ks[i] = ks[i];
    g.vs[i] = vs[i];
    g.os[i] = os[i];
  }
  g.B = B; g.H = H; g.Sq = Sq; g.Sk = Sk; g.D = D;
  g.q_scale = q_scale;
  g.causal = causal ? 1 : 0;
  g.o_dtype = o_dtype;
  // Vector key/value loads need unit d-stride, 16-byte aligned rows and a full
  // head dim; the batch/head offsets keep rows aligned when their strides do.
  auto kvec_ok = [&](int64_t dm) {
    return ks[3] == 1 && vs[3] == 1 && D == dm && (ks[2] * 2) % 16 == 0 && (vs[2] * 2) % 16 == 0 &&
           (ks[1] * 2) % 16 == 0 && (vs[1] * 2) % 16 == 0 && (ks[0] * 2) % 16 == 0 && (vs[0] * 2) % 16 == 0 &&
           (uintptr_t)k % 16 == 0 && (uintptr_t)v % 16 == 0 && qs[3] == 1 && (qs[2] * 2) % 16 == 0 &&
           (qs[1] * 2) % 16 == 0 && (qs[0] * 2) % 16 == 0 && (uintptr_t)q % 16 == 0;
  };
  // The fast kernel addresses a head's keys with 32-bit buffer offsets (up to two tiles
  // past the end) and positions with 32-bit integers.
  constexpr int NW = 8;  // waves of 32 queries per workgroup of the fast kernel
  // The fast kernel also takes a head dim below its 64 or 128 (a multiple of 8, padded with
  // zeros): 16-byte row vectors need only unit d-stride and aligned rows.
  auto rows_ok = [&]() {  // (row strides non-negative: a head's keys are addressed with unsigned buffer offsets)
    return ks[3] == 1 && vs[3] == 1 && qs[3] == 1 && D % 8 == 0 && ks[2] >= 0 && vs[2] >= 0 && qs[2] >= 0 &&
           (ks[2] * 2) % 16 == 0 && (vs[2] * 2) % 16 == 0 &&
           (qs[2] * 2) % 16 == 0 && (ks[1] * 2) % 16 == 0 && (vs[1] * 2) % 16 == 0 && (qs[1] * 2) % 16 == 0 &&
           (ks[0] * 2) % 16 == 0 && (vs[0] * 2) % 16 == 0 && (qs[0] * 2) % 16 == 0 && (uintptr_t)k % 16 == 0 &&
           (uintptr_t)v % 16 == 0 && (uintptr_t)q % 16 == 0;
  };
  auto fast_ok = [&](int64_t dm) {
    return rows_ok() && D <= dm && (Sk + 2 * AT_BN) * ks[2] * 2 < 0x7fffffffLL &&
           (Sk + 2 * AT_BN) * vs[2] * 2 < 0x7fffffffLL && Sq + NW * 32 < 0x7fffffffLL && Sk > 0;
  };
  const int64_t dm = D <= 64 ? 64 : 128;
  const bool fast_fits = fast_ok(dm), pipe_fits = D == 128 && fast_fits;
  if ((config == 1 && !pipe_fits) || (config == 2 && !fast_fits)) return NT_ERR_INVALID;
  // The eight-wave kernel is the default: measured on MI355X at B=4, H=32, S=4096, D=128
  // it runs 1,090-1,130 us non-causal against 1,140-1,270 us for the pipelined kernel.  Up
  // to 128 queries a head with at least 512 heads (B H), the four-wave kernel's 128-query
  // blocks waste half or less of what the eight-wave kernel's 256 do while the heads alone
  // fill the chip: [16,32,64,4096,128] 250 against 302 us, [32,32,32,4096,128] 452 against
  // 556 (fp16, interleaved medians); with fewer heads or longer queries the eight-wave one
  // wins ([4,32,128,4096,128] 120 against 144, [16,32,256,4096,128] 347 against 472).
  const bool pipe = config == 1;
  const bool few_queries = Sq <= AT_BM && B * H >= 512;
  const bool fast = config == 2 || (config == 0 && fast_fits && !few_queries);
  static_assert(ap::BM == NW * 32, "both fast kernels take 256 queries per workgroup");
  const int64_t bm = pipe || fast ? NW * 32 : AT_BM;
  const int64_t qblocks = cdiv(Sq, bm);
  if (qblocks * B * H > 0x7fffffffLL) return NT_ERR_INVALID;
  g.q_blocks = (int)qblocks;
  const dim3 grid((unsigned)(qblocks * B * H)), blk(AT_THREADS);
  if (pipe) {
    hipLaunchKernelGGL((attention_pipe_kernel<T>), grid, dim3(ap::NW * 64), 0, stream, g);
  } else if (fast) {
    if (dm == 64)
      hipLaunchKernelGGL((attention_fast_kernel<T, 64, NW>), grid, dim3(NW * 64), 0, stream, g);
    else
      hipLaunchKernelGGL((attention_fast_kernel<T, 128, NW>), grid, dim3(NW * 64), 0, stream, g);
  } else if (dm == 64) {
    if (kvec_ok(64))
      hipLaunchKernelGGL((attention_kernel<T, 64>), grid, blk, 0, stream, g);
    else
      hipLaunchKernelGGL((attention_generic_kernel<T, 64>), grid, blk, 0, stream, g);
  } else {
    if (kvec_ok(128))
      hipLaunchKernelGGL((attention_kernel<T, 128>), grid, blk, 0, stream, g);
    else
      hipLaunchKernelGGL((attention_generic_kernel<T, 128>), grid, blk, 0, stream, g);
  }
  return launch_status();
}

constexpr int AF_BN = 32;  // keys per tile
// fp32 inputs on the VALU: each query is held by LPQ lanes (1 for head dims up to 64, 2 up
// to 128), every lane with 64 of its dims of q and of the output accumulator, so a lane
// needs 128 registers for them and two waves fit each SIMD.  A wave's 64 lanes hold
// 64 / LPQ queries; the KS waves of a workgroup share those queries and take every KS-th
// 32-key tile each (KS 4 when there are few query blocks, so that short problems still
// spread over the CUs), then merge their running (max, sum, accumulator) states through
// LDS.  Each wave stages its own K and V tiles in LDS as [key][DM] rows and reads them
// with 16-byte broadcasts (4 FMAs per LDS read); the two halves of a query's dot product
// meet through one lane swap.  The q pre-scale and the rounding of p to the value type
// (fp32) are exact.
template <int DM, int KS>
__global__ __launch_bounds__(64 * KS) void attention_f32_kernel(AttnArgs g) {
  constexpr int LPQ = DM / 64, QPW = 64 / LPQ;  // lanes per query, queries per workgroup
  constexpr int TILE = AF_BN * DM;              // floats of one K (or V) tile
  constexpr int RED = (KS - 1) * 64 * 66;       // merge area: per lane acc[64], m, l
  constexpr int LDS = 2 * KS * TILE > RED ? 2 * KS * TILE : RED;
  __shared__ __attribute__((aligned(16))) float lds[LDS];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int qi = lane / LPQ, part = lane % LPQ;  // query of this lane, and which 64 dims
  float* sK = lds + w * 2 * TILE;
  float* sV = sK + TILE;
  int qb;
  int64_t bh;
  block_order(g, blockIdx.x, qb, bh);
  const int64_t b = bh / g.H, h = bh % g.H;
  const int64_t q0 = (int64_t)qb * QPW, qpos = q0 + qi;
  const float* Q = (const float*)g.q + b * g.qs[0] + h * g.qs[1];
  const float* K = (const float*)g.k + b * g.ks[0] + h * g.ks[1];
  const float* V = (const float*)g.v + b * g.vs[0] + h * g.vs[1];
  const int D = (int)g.D, d0 = part * 64;
  float qv[64], acc[64];
#pragma unroll
  for (int d = 0; d < 64; ++d) {
    qv[d] = (qpos < g.Sq && d0 + d < D) ? Q[qpos * g.qs[2] + (d0 + d) * g.qs[3]] * g.q_scale : 0.f;
    acc[d] = 0.f;
  }
  float m_i = -INFINITY, l_i = 0.f;
  int64_t nkt = cdiv(g.Sk, AF_BN);
  if (g.causal) {
    const int64_t last = (q0 + QPW - 1) / AF_BN + 1;
    if (last < nkt) nkt = last;
  }
  const bool kvec = g.ks[3] == 1 && g.vs[3] == 1 && D % 4 == 0 && g.ks[2] % 4 == 0 && g.vs[2] % 4 == 0 &&
                    ((uintptr_t)K & 15) == 0 && ((uintptr_t)V & 15) == 0;
  for (int64_t kt = w; kt < nkt; kt += KS) {
    const int64_t k0 = kt * AF_BN;
    wave_lds_order();  // this wave's reads of the previous tile come first
    if (kvec) {
      for (int e = lane; e < AF_BN * DM / 4; e += 64) {
        const int key = e / (DM / 4), d = (e % (DM / 4)) * 4;
        const int64_t kp = k0 + key;
        const bool ok = kp < g.Sk && d < D;
        *(float4*)(sK + key * DM + d) = ok ? *(const float4*)(K + kp * g.ks[2] + d) : float4{0.f, 0.f, 0.f, 0.f};
        *(float4*)(sV + key * DM + d) = ok ? *(const float4*)(V + kp * g.vs[2] + d) : float4{0.f, 0.f, 0.f, 0.f};
      }
    } else {
      for (int e = lane; e < AF_BN * DM; e += 64) {
        const int key = e / DM, d = e % DM;
        const int64_t kp = k0 + key;
        const bool ok = kp < g.Sk && d < D;
        sK[key * DM + d] = ok ? K[kp * g.ks[2] + d * g.ks[3]] : 0.f;
        sV[key * DM + d] = ok ? V[kp * g.vs[2] + d * g.vs[3]] : 0.f;
      }
    }
    wave_lds_order();  // every lane's writes before any lane reads
    float sc[AF_BN];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < AF_BN; ++j) {
      float dot = 0.f;
#pragma unroll
      for (int d = 0; d < 64; d += 4) {
        const float4 kv = *(const float4*)(sK + j * DM + d0 + d);
        dot = fmaf(qv[d], kv.x, dot);
        dot = fmaf(qv[d + 1], kv.y, dot);
        dot = fmaf(qv[d + 2], kv.z, dot);
        dot = fmaf(qv[d + 3], kv.w, dot);
      }
      if constexpr (LPQ == 2) dot += __shfl_xor(dot, 1, 64);
      const int64_t key = k0 + j;
      if (key >= g.Sk || (g.causal && qpos < key)) dot = -INFINITY;
      sc[j] = dot;
      mx = fmaxf(mx, dot);
    }
    const float m_new = fmaxf(m_i, mx);
    if (m_new != -INFINITY) {  // a tile of masked keys (so far) adds nothing
      const float alpha = __builtin_amdgcn_exp2f(m_i - m_new);
      float lsum = 0.f;
#pragma unroll
      for (int d = 0; d < 64; ++d) acc[d] *= alpha;
#pragma unroll
      for (int j = 0; j < AF_BN; ++j) {
        const float p = __builtin_amdgcn_exp2f(sc[j] - m_new);
        lsum += p;
#pragma unroll
        for (int d = 0; d < 64; d += 4) {
          const float4 vv = *(const float4*)(sV + j * DM + d0 + d);
          acc[d] = fmaf(p, vv.x, acc[d]);
          acc[d + 1] = fmaf(p, vv.y, acc[d + 1]);
          acc[d + 2] = fmaf(p, vv.z, acc[d + 2]);
          acc[d + 3] = fmaf(p, vv.w, acc[d + 3]);
        }
      }
      l_i = l_i * alpha + lsum;
      m_i = m_new;
    }
  }
  if constexpr (KS > 1) {
    // Merge: waves 1.. park their states, wave 0 rescales every state to the common max.
    __syncthreads();  // every wave is done with its tiles (the area is reused)
    if (w > 0) {
      float* r = lds + ((w - 1) * 64 + lane) * 66;
#pragma unroll
      for (int d = 0; d < 64; ++d) r[d] = acc[d];
      r[64] = m_i;
      r[65] = l_i;
    }
    __syncthreads();
    if (w > 0) return;
#pragma unroll
    for (int ww = 1; ww < KS; ++ww) {
      const float* r = lds + ((ww - 1) * 64 + lane) * 66;
      const float m2 = r[64], l2 = r[65];
      if (m2 == -INFINITY) continue;  // that wave saw only masked keys
      const float m = fmaxf(m_i, m2);
      const float a1 = m_i == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_i - m), a2 = __builtin_amdgcn_exp2f(m2 - m);
#pragma unroll
      for (int d = 0; d < 64; ++d) acc[d] = acc[d] * a1 + r[d] * a2;
      l_i = l_i * a1 + l2 * a2;
      m_i = m;
    }
  }
  if (qpos < g.Sq) {
    const float inv = 1.0f / l_i;
    const int64_t obase = b * g.os[0] + h * g.os[1] + qpos * g.os[2];
#pragma unroll
    for (int d = 0; d < 64; ++d)
      if (d0 + d < D) store_from_float(g.o, obase + (d0 + d) * g.os[3], g.o_dtype, acc[d] * inv);
  }
}

static int attention_f32_launch(const void* q, const int64_t* qs, const void* k, const int64_t* ks, const void* v,
                                const int64_t* vs, void* o, const int64_t* os, int o_dtype, int64_t B, int64_t H,
                                int64_t Sq, int64_t Sk, int64_t D, float q_scale, int causal, hipStream_t stream) {
  if (B < 0 || H < 0 || Sq < 0 || Sk < 0 || D < 0 || D > 128) return NT_ERR_INVALID;
  if (!valid_dtype(o_dtype)) return NT_ERR_INVALID;
  if (B * H * Sq * D == 0) return 0;
  if (!o || !os) return NT_ERR_INVALID;
  if (Sk == 0) return attention_empty_keys(o, os, o_dtype, B, H, Sq, D, stream);
  if (!q || !k || !v || !qs || !ks || !vs) return NT_ERR_INVALID;
  AttnArgs g{};
  g.q = q; g.k = k; g.v = v; g.o = o;
  for (int i = 0; i < 4; ++i) {
    g.qs[i] = qs[i];
    g.ks[i] = ks[i];
    g.vs[i] = vs[i];
    g.os[i] = os[i];
  }
  g.B = B; g.H = H; g.Sq = Sq; g.Sk = Sk; g.D = D;
  g.q_scale = q_scale;
  g.causal = causal ? 1 : 0;
  g.o_dtype = o_dtype;
  // Four waves splitting the keys of each query block when there are fewer than 512 blocks.
  const int64_t lpq = D <= 64 ? 1 : 2;
  const int64_t qblocks = cdiv(Sq, 64 / lpq);
  if (qblocks * B * H > 0x7fffffffLL) return NT_ERR_INVALID;
  g.q_blocks = (int)qblocks;
  const bool split = qblocks * B * H < 512;
  const dim3 grid((unsigned)(qblocks * B * H));
  if (D <= 64 && split)
    hipLaunchKernelGGL((attention_f32_kernel<64, 4>), grid, dim3(256), 0, stream, g);
  else if (D <= 64)
    hipLaunchKernelGGL((attention_f32_kernel<64, 1>), grid, dim3(64), 0, stream, g);
  else if (split)
    hipLaunchKernelGGL((attention_f32_kernel<128, 4>), grid, dim3(256), 0, stream, g);
  else
    hipLaunchKernelGGL((attention_f32_kernel<128, 1>), grid, dim3(64), 0, stream, g);
  return launch_status();
}

}  // namespace nt

#define NT_ATTN_PARAMS                                                                                             \
  const void *q, const int64_t *qs, const void *k, const int64_t *ks, const void *v, const int64_t *vs, void *o,  \
      const int64_t *os, int o_dtype, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D, float q_scale,     \
      int causal, hipStream_t stream
#define NT_ATTN_ARGS q, qs, k, ks, v, vs, o, os, o_dtype, B, H, Sq, Sk, D, q_scale, causal, stream

extern "C" int nt_attention_f16(NT_ATTN_PARAMS) { return nt::attention_launch<nt::f16_t>(NT_ATTN_ARGS); }
extern "C" int nt_attention_bf16(NT_ATTN_PARAMS) { return nt::attention_launch<nt::bf16_t>(NT_ATTN_ARGS); }
extern "C" int nt_attention_f32(NT_ATTN_PARAMS) { return nt::attention_f32_launch(NT_ATTN_ARGS); }
extern "C" int nt_attention_config_f16(NT_ATTN_PARAMS, int config) {
  return nt::attention_launch<nt::f16_t>(NT_ATTN_ARGS, config);
}
extern "C" int nt_attention_config_bf16(NT_ATTN_PARAMS, int config) {
  return nt::attention_launch<nt::bf16_t>(NT_ATTN_ARGS, config);
}
