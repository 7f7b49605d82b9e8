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
  const uint16_t* Q = (const uint16_t*)g.q + b * g.qs[0] + h * g.qs[1];

  // Q^T fragments of this lane's queries (one per block), pre-scaled and rounded to the
  // input type.
  int qpos[QB];
  frag qf[QB][G::DSUB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    qpos[qb] = qw + qb * 32 + (lane & 31);
#pragma unroll
    for (int dd = 0; dd < G::DSUB; ++dd) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (qpos[qb] < g.Sq) raw = *(const u32x4*)(Q + (int64_t)qpos[qb] * g.qs[2] + dd * 16 + half * 8);
      uint16_t tmp[8];
      const uint16_t* hv = (const uint16_t*)&raw;
#pragma unroll
      for (int u = 0; u < 8; ++u) tmp[u] = elem<T>::from_float(elem<T>::to_float(hv[u]) * g.q_scale);
      qf[qb][dd] = __builtin_bit_cast(frag, *(const u32x4*)tmp);
    }
  }

  // Tile loaders, 256 lanes per operand: with four waves every lane fetches both K and V;
  // with eight, waves 0-3 fetch K and waves 4-7 fetch V (lane index lt within the 256).
  // K: load i brings key i * KEYS_PER_LOAD + kr, chunk kc.  V: a 4 (key) x 8 (d) block,
  // keys 4 kq .. 4 kq + 3, d 8 db .. 8 db + 7 (lanes with db >= DM / 8 idle when DM = 64).
  const int lt = tid & (AT_THREADS - 1);
  const bool k_role = NW == 4 || wave < 4;
  const bool v_role = (NW == 4 || wave >= 4) && (lt >> 4) < DM / 8;
  const int ks2b = (int)g.ks[2] * 2, vs2b = (int)g.vs[2] * 2;
  const __amdgpu_buffer_rsrc_t rsK = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint16_t*)g.k + b * g.ks[0] + h * g.ks[1]), (short)0, (Sk - 1) * ks2b + DM * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsV = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint16_t*)g.v + b * g.vs[0] + h * g.vs[1]), (short)0, (Sk - 1) * vs2b + DM * 2, 0x00020000);
  const int kr = lt / G::CPR, kc = lt % G::CPR;
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
        rk[i] = __builtin_amdgcn_raw_buffer_load_b128(rsK, vK, (k0 + i * G::KEYS_PER_LOAD) * ks2b, 0);
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

  if (nkt > 0) {
    load_tile(0);
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
      __syncthreads();
#pragma unroll
      for (int e0 = 0; e0 < 32 * 16; e0 += 64) {
        const int e = e0 + lane;
        const int row = e >> 4, grp = (e & 15) * 4;
        const int qp = qw + qb * 32 + row;
        if (qp < g.Sq) {
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
      __syncthreads();
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

template <typename T>
static int attention_launch(const void* q, const int64_t* qs, const void* k, const int64_t* ks, const void* v,
                            const int64_t* vs, void* o, const int64_t* os, int o_dtype, int64_t B, int64_t H,
                            int64_t Sq, int64_t Sk, int64_t D, float q_scale, int causal, hipStream_t stream) {
  if (B < 0 || H < 0 || Sq < 0 || Sk < 0 || D < 0 || D > 128) return NT_ERR_INVALID;
  if (!valid_dtype(o_dtype)) return NT_ERR_INVALID;
  if (B * H * Sq * D == 0) return 0;
  if (!q || !k || !v || !o || !qs || !ks || !vs || !os) return NT_ERR_INVALID;
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
  auto fast_ok = [&](int64_t dm) {
    return kvec_ok(dm) && (Sk + 2 * AT_BN) * ks[2] * 2 < 0x7fffffffLL && (Sk + 2 * AT_BN) * vs[2] * 2 < 0x7fffffffLL &&
           Sq + NW * 32 < 0x7fffffffLL && Sk > 0;
  };
  const int64_t dm = D <= 64 ? 64 : 128;
  const bool fast = fast_ok(dm);
  const int64_t bm = fast ? NW * 32 : AT_BM;
  const int64_t qblocks = cdiv(Sq, bm);
  if (qblocks * B * H > 0x7fffffffLL) return NT_ERR_INVALID;
  g.q_blocks = (int)qblocks;
  const dim3 grid((unsigned)(qblocks * B * H)), blk(AT_THREADS);
  if (fast) {
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

// fp32 inputs: one lane per query, VALU dot products against key/value tiles staged
// in LDS (every lane reads the same key, an LDS broadcast).  The q pre-scale and the
// rounding of p to the value type are exact in fp32.
constexpr int AF_Q = 64, AF_BN = 32;

__global__ __launch_bounds__(AF_Q) void attention_f32_kernel(AttnArgs g) {
  __shared__ float sK[AF_BN][128];
  __shared__ float sV[AF_BN][128];
  const int tid = threadIdx.x;
  int qb;
  int64_t bh;
  block_order(g, blockIdx.x, qb, bh);
  const int64_t b = bh / g.H, h = bh % g.H;
  const int64_t q0 = (int64_t)qb * AF_Q, qpos = q0 + tid;
  const float* Q = (const float*)g.q + b * g.qs[0] + h * g.qs[1];
  const float* K = (const float*)g.k + b * g.ks[0] + h * g.ks[1];
  const float* V = (const float*)g.v + b * g.vs[0] + h * g.vs[1];
  const int D = (int)g.D;
  float qv[128], acc[128];
#pragma unroll
  for (int d = 0; d < 128; ++d) {
    qv[d] = (qpos < g.Sq && d < D) ? Q[qpos * g.qs[2] + d * g.qs[3]] * g.q_scale : 0.f;
    acc[d] = 0.f;
  }
  float m_i = -INFINITY, l_i = 1.0f;
  int64_t nkt = cdiv(g.Sk, AF_BN);
  if (g.causal) {
    const int64_t last = (q0 + AF_Q - 1) / AF_BN + 1;
    if (last < nkt) nkt = last;
  }
  for (int64_t kt = 0; kt < nkt; ++kt) {
    const int64_t k0 = kt * AF_BN;
    for (int e = tid; e < AF_BN * 128; e += AF_Q) {
      const int key = e / 128, d = e % 128;
      const int64_t kp = k0 + key;
      const bool ok = kp < g.Sk && d < D;
      sK[key][d] = ok ? K[kp * g.ks[2] + d * g.ks[3]] : 0.f;
      sV[key][d] = ok ? V[kp * g.vs[2] + d * g.vs[3]] : 0.f;
    }
    __syncthreads();
    float s[AF_BN];
    float mx = -INFINITY;
    for (int j = 0; j < AF_BN; ++j) {
      float dot = 0.f;
#pragma unroll
      for (int d = 0; d < 128; ++d) dot = fmaf(qv[d], sK[j][d], dot);
      const int64_t key = k0 + j;
      if (key >= g.Sk || (g.causal && qpos < key)) dot = -INFINITY;
      s[j] = dot;
      mx = fmaxf(mx, dot);
    }
    const float m_new = fmaxf(m_i, mx);
    const float alpha = __builtin_amdgcn_exp2f(m_i - m_new);
    float lsum = 0.f;
#pragma unroll
    for (int d = 0; d < 128; ++d) acc[d] *= alpha;
    for (int j = 0; j < AF_BN; ++j) {
      const float p = __builtin_amdgcn_exp2f(s[j] - m_new);
      lsum += p;
#pragma unroll
      for (int d = 0; d < 128; ++d) acc[d] = fmaf(p, sV[j][d], acc[d]);
    }
    l_i = l_i * alpha + lsum;
    m_i = m_new;
    __syncthreads();
  }
  if (qpos < g.Sq) {
    const float inv = 1.0f / l_i;
    const int64_t obase = b * g.os[0] + h * g.os[1] + qpos * g.os[2];
#pragma unroll
    for (int d = 0; d < 128; ++d)
      if (d < D) store_from_float(g.o, obase + d * g.os[3], g.o_dtype, acc[d] * inv);
  }
}

static int attention_f32_launch(const void* q, const int64_t* qs, const void* k, const int64_t* ks, const void* v,
                                const int64_t* vs, void* o, const int64_t* os, int o_dtype, int64_t B, int64_t H,
                                int64_t Sq, int64_t Sk, int64_t D, float q_scale, int causal, hipStream_t stream) {
  if (B < 0 || H < 0 || Sq < 0 || Sk < 0 || D < 0 || D > 128) return NT_ERR_INVALID;
  if (!valid_dtype(o_dtype)) return NT_ERR_INVALID;
  if (B * H * Sq * D == 0) return 0;
  if (!q || !k || !v || !o || !qs || !ks || !vs || !os) return NT_ERR_INVALID;
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
  const int64_t qblocks = cdiv(Sq, AF_Q);
  if (qblocks * B * H > 0x7fffffffLL) return NT_ERR_INVALID;
  g.q_blocks = (int)qblocks;
  hipLaunchKernelGGL(attention_f32_kernel, dim3((unsigned)(qblocks * B * H)), dim3(AF_Q), 0, stream, g);
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
