// mcpm_kernels.hip -- gfx950 kernels of the decode path.
//
// Numerics contract (the CPU oracle follows the same sequences):
//  * Q4_K/Q6_K x Q8_K dots form, per 256-block, the eight int32 lane sums of
//    the reference's AVX2 kernels (src/ops/ops_avx2.cpp:161-181, 224-270):
//    lane m folds bytes 4m..4m+3 of every 32-byte group.  Per row, lane m then
//    runs acc_m = fma(d_x*d_w, float(isum_m), acc_m) over blocks in order,
//    Q4_K adds acc_min = fma(-(d_x*dmin_w), float(minsum), acc_min), and the
//    lanes are summed ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) (ops_avx2.cpp:43-48).
//    The result is bit-identical to the reference's compiled AVX2 GEMV.
//  * Q8_K quantization: d = amax*(1/127), v = x*(127/amax), rint or round.
//  * Sums of squares: 256 strided partials, then a pairwise tree.
//  * Everything is compiled with -ffp-contract=off; fused multiply-adds are
//    explicit.
#include <algorithm>

#include <cstdlib>

#include "mcpm_attn.h"
#include "mcpm_device.h"

namespace mcpm {

// ------------------------------------------------------- standalone ops ----

// Q8_K blocks of an fp32 vector (optionally RMS-normalised) in native layout.
// mode: PRO_QUANT_EVEN / PRO_QUANT_AWAY / PRO_NORM_AWAY / PRO_NORM_EVEN.
__global__ void __launch_bounds__(256) k_quantize_q8k(const float* __restrict__ x, const float* __restrict__ gamma,
                                                      float eps, int dim, int mode, BlockQ8K* __restrict__ out) {
  __shared__ float red[260];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const bool norm = (mode == PRO_NORM_AWAY || mode == PRO_NORM_EVEN);
  const bool away = (mode == PRO_QUANT_AWAY || mode == PRO_NORM_AWAY);
  float rms = 1.0f;
  if (norm) rms = block_rms_scale(x, dim, eps, red);
  const int nb = dim / QK_K;
  for (int b = wave; b < nb; b += 4) {
    const float4 xv = reinterpret_cast<const float4*>(x + b * QK_K)[lane];
    float v[4] = {xv.x, xv.y, xv.z, xv.w};
    if (norm) {
      const float4 gv = reinterpret_cast<const float4*>(gamma + b * QK_K)[lane];
      v[0] = (v[0] * rms) * gv.x;
      v[1] = (v[1] * rms) * gv.y;
      v[2] = (v[2] * rms) * gv.z;
      v[3] = (v[3] * rms) * gv.w;
    }
    uint32_t packed;
    float d;
    int gsum;
    quant_block_wave(v, away, packed, d, gsum);
    reinterpret_cast<uint32_t*>(out[b].qs)[lane] = packed;
    if ((lane & 3) == 0) out[b].bsums[lane >> 2] = static_cast<int16_t>(gsum);
    if (lane == 0) out[b].d = d;
  }
}

hipError_t launch_quantize_q8k(const float* x, const float* gamma, float eps, int dim, int mode, BlockQ8K* out,
                               hipStream_t s) {
  hipLaunchKernelGGL(k_quantize_q8k, dim3(1), dim3(256), 0, s, x, gamma, eps, dim, mode, out);
  return hipGetLastError();
}

// rmsnorm (src/ops/ops.cpp:468-481): out = (x*rms)*w.
__global__ void __launch_bounds__(256) k_rmsnorm(const float* __restrict__ x, const float* __restrict__ w, float eps,
                                                 int dim, float* __restrict__ out) {
  __shared__ float red[260];
  const float rms = block_rms_scale(x, dim, eps, red);
  for (int i = threadIdx.x; i < dim; i += 256) out[i] = (x[i] * rms) * w[i];
}

hipError_t launch_rmsnorm(const float* x, const float* w, float eps, int dim, float* out, hipStream_t s) {
  hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(256), 0, s, x, w, eps, dim, out);
  return hipGetLastError();
}

// swiglu_and_quantize_q8k (src/ops/ops.cpp:725-765): dim/256 blocks, lround.
__global__ void __launch_bounds__(256) k_swiglu_quant(const float* __restrict__ g, const float* __restrict__ u, int dim,
                                                      BlockQ8K* __restrict__ out) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nb = dim / QK_K;
  for (int b = wave; b < nb; b += 4) {
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = b * QK_K + 4 * lane + k;
      const float gg = g[i];
      const float silu = gg / (1.0f + exp_f32(-gg));
      v[k] = silu * u[i];
    }
    uint32_t packed;
    float d;
    int gsum;
    quant_block_wave(v, true, packed, d, gsum);
    reinterpret_cast<uint32_t*>(out[b].qs)[lane] = packed;
    if ((lane & 3) == 0) out[b].bsums[lane >> 2] = static_cast<int16_t>(gsum);
    if (lane == 0) out[b].d = d;
  }
}

hipError_t launch_swiglu_quant(const float* g, const float* u, int dim, BlockQ8K* out, hipStream_t s) {
  hipLaunchKernelGGL(k_swiglu_quant, dim3(1), dim3(256), 0, s, g, u, dim, out);
  return hipGetLastError();
}

// apply_rope for every head with a host-built (cos, sin) row for pos.
__global__ void k_rope(float* __restrict__ vec, const float2* __restrict__ cs, int n_pairs, int half_hd) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n_pairs) return;
  const float2 c = cs[p % half_hd];
  const float v0 = vec[2 * p], v1 = vec[2 * p + 1];
  vec[2 * p] = v0 * c.x - v1 * c.y;
  vec[2 * p + 1] = v0 * c.y + v1 * c.x;
}

hipError_t launch_rope(float* vec, const float2* cs, int n_heads, int head_dim, hipStream_t s) {
  const int n_pairs = n_heads * head_dim / 2;
  hipLaunchKernelGGL(k_rope, dim3((n_pairs + 255) / 256), dim3(256), 0, s, vec, cs, n_pairs, head_dim / 2);
  return hipGetLastError();
}

__global__ void k_kv_append(const float* __restrict__ k, const float* __restrict__ v, float* __restrict__ kc,
                            float* __restrict__ vc, const int* __restrict__ state, int kvd) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= kvd) return;
  const size_t pos = static_cast<size_t>(state[1]);
  kc[pos * kvd + i] = k[i];
  vc[pos * kvd + i] = v[i];
}

hipError_t launch_kv_append(const float* k, const float* v, float* kc, float* vc, const int* state, int kvd,
                            hipStream_t s) {
  hipLaunchKernelGGL(k_kv_append, dim3((kvd + 255) / 256), dim3(256), 0, s, k, v, kc, vc, state, kvd);
  return hipGetLastError();
}


// NT consecutive tokens (token k with context Tk[k], k < NT; every Tk[k] >
// c*ATTN_CHUNK) on one chunk: each token's sums are attn_token_chunk's, in
// the same order, and the tokens' chains run side by side, so each K and V
// value read from LDS serves NT tokens.  Token k's queries at sQ + k*QSZ, its
// softmax terms at sE + k*ESZ, its (m_c, z_c) at mz[k*ATTN_MAX_GROUP + hh], its
// outputs in o[k].
// GM: the most query heads per kv head that sQ and sE hold.  SWZ: K rows
// unpadded, 64 floats apart, float4 c4 of row j at (c4 ^ (j % 16)) (distinct
// banks across 16 rows read together, as the padding gives).  (m_c, z_c) go
// to put_mz(k, hh, value) from lane 0 of the head's wave.
template <int HDM, int OPT, int NT, bool WL, int GM, bool SWZ, class PutMZ>
__device__ __forceinline__ void attn_tokens_chunk(const float* sK, const float* sV, const float* sQ, float* sE,
                                                  PutMZ put_mz, int c, const int (&Tk)[NT], int group, int hd, int gh,
                                                  float scale, float (&o)[NT][OPT]) {
  constexpr int KS = SWZ ? HDM : HDM + 4;
  constexpr int QSZ = GM * HDM, ESZ = GM * ATTN_CHUNK;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // float offset of dimension i (a multiple of 4) in this lane's K row
  auto kof = [&](int i) { return SWZ ? (((i >> 2) ^ (lane & 15)) << 2) : i; };
  for (int hh = wave; hh < group; hh += 4) {
    const float* kt = &sK[lane * KS];
    const float* qh = sQ + hh * HDM;
    float dot[NT];
#pragma unroll
    for (int k = 0; k < NT; ++k) dot[k] = 0.0f;
    // the next 4 dimensions' K and q are read while this step's fmas run
    // (the last step reads itself again)
    f32x4 kc4 = *reinterpret_cast<const f32x4*>(kt + kof(0)), qc4[NT];
#pragma unroll
    for (int k = 0; k < NT; ++k) qc4[k] = *reinterpret_cast<const f32x4*>(qh + k * QSZ);
#pragma unroll 2
    for (int i = 0; i < hd; i += 4) {
      const int in = min(i + 4, hd - 4);
      const f32x4 kn4 = *reinterpret_cast<const f32x4*>(kt + kof(in));
      f32x4 qn4[NT];
#pragma unroll
      for (int k = 0; k < NT; ++k) qn4[k] = *reinterpret_cast<const f32x4*>(qh + k * QSZ + in);
#pragma unroll
      for (int k = 0; k < NT; ++k) {
        dot[k] = __builtin_fmaf(qc4[k].x, kc4.x, dot[k]);
        dot[k] = __builtin_fmaf(qc4[k].y, kc4.y, dot[k]);
        dot[k] = __builtin_fmaf(qc4[k].z, kc4.z, dot[k]);
        dot[k] = __builtin_fmaf(qc4[k].w, kc4.w, dot[k]);
      }
      kc4 = kn4;
#pragma unroll
      for (int k = 0; k < NT; ++k) qc4[k] = qn4[k];
    }
#pragma unroll
    for (int k = 0; k < NT; ++k) {
      const bool present = c * ATTN_CHUNK + lane < Tk[k];
      const float sv = present ? dot[k] * scale : -1e9f;
      const float mc = fmaxf(wave_max_fast(sv), -1e9f);
      const float e = present ? exp_f32(sv - mc) : 0.0f;
      const float z = wave_tree_sum_fast(e);
      sE[k * ESZ + hh * ATTN_CHUNK + lane] = e;
      if (lane == 0) put_mz(k, hh, make_float2(mc, z));
    }
  }
  // WL (head_dim 64): the weighted sums of head hh run on the wave that
  // formed its softmax terms, so a wave-level ordering suffices
  if constexpr (WL) wave_sync();
  else __syncthreads();
  // positions 0..nt_k-1 for token k: the first nt_lo for every token, then
  // the later ones for the tokens that have them
  int nt[NT];
#pragma unroll
  for (int k = 0; k < NT; ++k) nt[k] = min(ATTN_CHUNK, Tk[k] - c * ATTN_CHUNK);
  int nt_lo = nt[0], nt_hi = nt[0];
#pragma unroll
  for (int k = 1; k < NT; ++k) {
    nt_lo = min(nt_lo, nt[k]);
    nt_hi = max(nt_hi, nt[k]);
  }
#pragma unroll
  for (int u = 0; u < OPT; ++u) {
    const int oi = tid + 256 * u;
    float acc[NT];
#pragma unroll
    for (int k = 0; k < NT; ++k) acc[k] = 0.0f;
    if (oi < gh) {
      const int hh = oi / hd, i = oi - hh * hd;
      const float* eh = &sE[hh * ATTN_CHUNK];
      // positions in groups of 4, the next group's softmax terms and V
      // values read while this group's fmas run, then the rest one by one
      const int n4 = nt_lo & ~3;
      if (n4 > 0) {
        auto ld4 = [&](int j0, f32x4 (&e4)[NT], f32x4& v4) {
#pragma unroll
          for (int k = 0; k < NT; ++k) e4[k] = *reinterpret_cast<const f32x4*>(eh + k * ESZ + j0);
          v4 = f32x4{sV[j0 * HDM + i], sV[(j0 + 1) * HDM + i], sV[(j0 + 2) * HDM + i], sV[(j0 + 3) * HDM + i]};
        };
        f32x4 ec[NT], vcur;
        ld4(0, ec, vcur);
#pragma unroll 2
        for (int j0 = 0; j0 < n4; j0 += 4) {
          f32x4 en[NT], vnx;
          ld4(min(j0 + 4, n4 - 4), en, vnx);
#pragma unroll
          for (int k = 0; k < NT; ++k) {
            acc[k] = __builtin_fmaf(ec[k].x, vcur.x, acc[k]);
            acc[k] = __builtin_fmaf(ec[k].y, vcur.y, acc[k]);
            acc[k] = __builtin_fmaf(ec[k].z, vcur.z, acc[k]);
            acc[k] = __builtin_fmaf(ec[k].w, vcur.w, acc[k]);
          }
          vcur = vnx;
#pragma unroll
          for (int k = 0; k < NT; ++k) ec[k] = en[k];
        }
      }
      for (int j = n4; j < nt_lo; ++j) {
        const float v = sV[j * HDM + i];
#pragma unroll
        for (int k = 0; k < NT; ++k) acc[k] = __builtin_fmaf(eh[k * ESZ + j], v, acc[k]);
      }
      for (int j = nt_lo; j < nt_hi; ++j) {
        const float v = sV[j * HDM + i];
#pragma unroll
        for (int k = 0; k < NT; ++k)
          if (j < nt[k]) acc[k] = __builtin_fmaf(eh[k * ESZ + j], v, acc[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < NT; ++k) o[k][u] = acc[k];
  }
}

template <int HDM, bool WL>
__global__ void __launch_bounds__(256) k_attention(const float* __restrict__ q, const float* __restrict__ kc,
                                                   const float* __restrict__ vc, const int* __restrict__ state,
                                                   int n_heads, int n_kv_heads, int hd, int max_chunks,
                                                   float* __restrict__ part_o, float2* __restrict__ part_mz,
                                                   int pos0, size_t tok_q, size_t tok_o, size_t tok_mz) {
  __shared__ __attribute__((aligned(16))) float lds[AttnLds<HDM>::bytes / sizeof(float)];
  // decode: the position from the step state; prefill (pos0 >= 0): token
  // blockIdx.z at position pos0 + z, with its own q and partials
  int T;
  if (pos0 >= 0) {
    T = pos0 + static_cast<int>(blockIdx.z) + 1;
    q += blockIdx.z * tok_q;
    part_o += blockIdx.z * tok_o;
    part_mz += blockIdx.z * tok_mz;
  } else {
    T = state[1] + 1;
  }
  AttnRegs<HDM / 16> R;
  attn_split<HDM, false, WL>(q, kc, vc, T, static_cast<int>(blockIdx.x), static_cast<int>(blockIdx.y), n_heads,
                         n_kv_heads, hd, max_chunks, part_o, part_mz, AttnLds<HDM>(lds), R, false);
}

static_assert(ATTN_Q8K_MAX_CHUNKS == ATTN_CPW, "one work group holds every chunk's o_c in registers");

// Decode, contexts of at most ATTN_CPW chunks, head_dim 64: one work group of
// four 256-thread groups per kv head.  Group g runs chunks g and g + 4 (the
// splits' arithmetic, attn_token_chunk on its own staged K and V rows; the
// query rows are shared), the groups' waves sharing each SIMD; then the work
// group combines the chunks with the consumers' arithmetic (m = max m_c;
// f_c = exp(m_c - m); Z = fma(z_c, f_c, Z); O = fma(o_c, f_c, O); O / Z) and
// quantizes its heads' outputs ties-even into Q8_K blocks (the group's
// gh = group*64 values are gh/256 whole blocks: block kvh*gh/256 + r), so
// the O projection reads them as they are.  A longer context sets *err and
// writes nothing.
constexpr int AQ_GROUPS = 4;
struct AttnQ8kLds {
  static constexpr int K = ATTN_CHUNK * 68, V = ATTN_CHUNK * 64, E = ATTN_MAX_GROUP * ATTN_CHUNK;
  static constexpr int PER = K + V + E;                        // floats per group
  static constexpr int Q = ATTN_MAX_GROUP * 64;
  static constexpr int MZ = ATTN_CPW * ATTN_MAX_GROUP;        // float2
  static constexpr size_t bytes = (AQ_GROUPS * PER + Q) * sizeof(float) + MZ * sizeof(float2);
};

__global__ void __launch_bounds__(256 * AQ_GROUPS) k_attention_q8k(const float* __restrict__ q,
                                                                   const float* __restrict__ kc,
                                                                   const float* __restrict__ vc,
                                                                   const int* __restrict__ state, int n_heads,
                                                                   int n_kv_heads, BlockQ8K* __restrict__ out,
                                                                   unsigned* __restrict__ err) {
  constexpr int HDM = 64, NV = HDM / 16, OPT = ATTN_MAX_GROUP * HDM / 256, KS = HDM + 4;
  using L = AttnQ8kLds;
  __shared__ __attribute__((aligned(16))) float lds[L::bytes / sizeof(float)];
  const int T = state[1] + 1;
  const int nch = (T + ATTN_CHUNK - 1) / ATTN_CHUNK;
  if (nch > ATTN_CPW) {  // uniform: before any barrier
    if (blockIdx.x == 0 && threadIdx.x == 0) *err = 1u;
    return;
  }
  const int tid = threadIdx.x, g = tid >> 8, t = tid & 255, kvh = blockIdx.x;
  const int hd = HDM, group = n_heads / n_kv_heads, gh = group * hd, kvd = n_kv_heads * hd;
  const int r4 = hd / 4, nf4 = ATTN_CHUNK * r4;
  const float scale = 1.0f / sqrtf(static_cast<float>(hd));
  const size_t head_off = static_cast<size_t>(kvh) * hd;
  float* sK = lds + g * L::PER;
  float* sV = sK + L::K;
  float* sE = sV + L::V;
  float* sQ = lds + AQ_GROUPS * L::PER;
  float2* sMZ = reinterpret_cast<float2*>(sQ + L::Q);
  AttnRegs<NV> R;
  if (g < nch) attn_load_chunk<NV>(R, kc, vc, g, T, kvd, head_off, r4, nf4, t);  // uniform in the group
  if (g == 0) {  // group 0 stages the queries for every group
    const float* qg = q + static_cast<size_t>(kvh) * gh;
#pragma unroll
    for (int u = 0; u < OPT; ++u) {
      const int i = min(t + 256 * u, gh - 1);  // threads past the queries store query gh-1 again
      sQ[(i / hd) * HDM + i % hd] = qg[i];
    }
  }
  const int rounds = (nch + AQ_GROUPS - 1) / AQ_GROUPS;  // 1 or 2
  float oc[2][OPT];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    if (r < rounds) {  // uniform
      // chunk c of group g; a group past the context (c >= nch, uniform in
      // the group) loads, stages and computes nothing and only keeps the
      // barriers
      const int c = g + AQ_GROUPS * r;
      __syncthreads();  // readers of the previous chunk are done
      if (c < nch) {
#pragma unroll
        for (int u = 0; u < NV; ++u) {
          const int f = min(t + 256 * u, nf4 - 1);
          const int j = f / r4, c4 = f - j * r4;
          *reinterpret_cast<f32x4*>(&sK[j * KS + c4 * 4]) = R.k[u];
          *reinterpret_cast<f32x4*>(&sV[j * HDM + c4 * 4]) = R.v[u];
        }
        if (c + AQ_GROUPS < nch) attn_load_chunk<NV>(R, kc, vc, c + AQ_GROUPS, T, kvd, head_off, r4, nf4, t);
      }
      __syncthreads();
      if (c < nch)
        attn_token_chunk<HDM, OPT, true>(sK, sV, sQ, sE, sMZ + c * ATTN_MAX_GROUP, c, T, group, hd, gh, scale, oc[r], t);
    }
  }
  // every chunk's o_c into the staging area (each group's own K rows: its
  // readers are done after the barrier), o_c of chunk c at sO[c*gh + oi]
  __syncthreads();
  float* sO = lds;  // ATTN_CPW * 512 floats at most: within group 0's K and V rows
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int c = g + AQ_GROUPS * r;
    if (r < rounds && c < nch) {
#pragma unroll
      for (int u = 0; u < OPT; ++u) {
        const int oi = t + 256 * u;
        if (oi < gh) sO[c * gh + oi] = oc[r][u];
      }
    }
  }
  __syncthreads();
  float* sX = lds + 2 * L::PER;  // group 2's area: gh floats
  if (tid < gh) {
    const int oi = tid, hh = oi / hd;
    float m = sMZ[hh].x;
    for (int cc = 1; cc < nch; ++cc) m = fmaxf(m, sMZ[cc * ATTN_MAX_GROUP + hh].x);
    float Z = 0.0f, O = 0.0f;
    for (int cc = 0; cc < nch; ++cc) {
      const float2 mz = sMZ[cc * ATTN_MAX_GROUP + hh];
      const float f = exp_f32(mz.x - m);
      Z = __builtin_fmaf(mz.y, f, Z);
      O = __builtin_fmaf(sO[cc * gh + oi], f, O);
    }
    sX[oi] = O / Z;
  }
  __syncthreads();
  // block r of the group on row r (16 lanes) of wave 0, lane j holding
  // values 16j .. 16j+15: the GEMV prologue's quantization
  const int row = tid >> 4, j = tid & 15;
  if (tid < 64 && 256 * row < gh) {
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 x4 = *reinterpret_cast<const f32x4*>(&sX[256 * row + 16 * j + 4 * i]);
      v[4 * i] = x4.x;
      v[4 * i + 1] = x4.y;
      v[4 * i + 2] = x4.z;
      v[4 * i + 3] = x4.w;
    }
    u32x4 packed;
    float d;
    int gsum;
    quant_block_row16(v, false, packed, d, gsum);
    BlockQ8K* blk = out + kvh * (gh / QK_K) + row;
    uint32_t* qs = reinterpret_cast<uint32_t*>(blk->qs) + 4 * j;  // 4-byte aligned
    qs[0] = packed.x;
    qs[1] = packed.y;
    qs[2] = packed.z;
    qs[3] = packed.w;
    blk->bsums[j] = static_cast<int16_t>(gsum);
    if (j == 0) blk->d = d;
  }
}

// Prefill: chunk blockIdx.y of kv head blockIdx.x for the tile of tt
// consecutive tokens from blockIdx.z * tt (token z at position pos0 + z,
// its own q and partials).  The chunk's K and V rows are staged once; the
// tile's tokens whose context reaches the chunk then run on it ATTN_TOK at a
// time (attn_tokens_chunk: for each token the arithmetic of k_attention's
// launch for that token) and write their partials for the chunk.  Rows the
// tile stages past a token's context take no part in that token's sums.
constexpr int ATTN_TOK = 4;

// WL (head_dim 64): every LDS value a wave reads in the token loop (its
// heads' queries, softmax terms and (m_c, z_c)) was written by the same wave,
// so the loop orders them within the wave and only the staged K/V rows wait
// for a work-group barrier.
template <int HDM, bool WL, int GM>
__global__ void __launch_bounds__(256) k_attention_tile(const float* __restrict__ q, const float* __restrict__ kc,
                                                        const float* __restrict__ vc, int n_heads, int n_kv_heads,
                                                        int hd, int max_chunks, float* __restrict__ part_o,
                                                        float2* __restrict__ part_mz, int pos0, int n_tok, int tt,
                                                        size_t tok_q, size_t tok_o, size_t tok_mz) {
  // GM 4 (head_dim 64, at most 4 query heads per kv head): sQ and sE for 4
  // heads, K rows unpadded and swizzled, (m_c, z_c) stored straight from
  // the wave: 40 KB of LDS, four work groups per CU where the padded layout
  // for 8 heads (50 KB) fits three
  constexpr bool SWZ = GM == 4;
  constexpr int NV = HDM / 16;
  constexpr int OPT = GM * HDM / 256;
  constexpr int NQ = GM * HDM / 256;
  constexpr int KS = SWZ ? HDM : HDM + 4;
  constexpr int NT = ATTN_TOK;
  constexpr int QSZ = GM * HDM, ESZ = GM * ATTN_CHUNK;
  static_assert(!SWZ || (WL && HDM == 64), "the compact layout is for head_dim 64");
  __shared__ __attribute__((aligned(16))) float sK[ATTN_CHUNK * KS];
  __shared__ __attribute__((aligned(16))) float sV[ATTN_CHUNK * HDM];
  __shared__ __attribute__((aligned(16))) float sQ[NT * QSZ];
  __shared__ __attribute__((aligned(16))) float sE[NT * ESZ];
  __shared__ float2 sMZ[SWZ ? 1 : NT * ATTN_MAX_GROUP];
  const int tid = threadIdx.x;
  const int kvh = blockIdx.x, c = blockIdx.y;
  const int z0 = static_cast<int>(blockIdx.z) * tt;
  const int zlo = max(z0, c * ATTN_CHUNK - pos0);  // first token with pos0 + z + 1 > c * ATTN_CHUNK
  const int zhi = min(z0 + tt, n_tok);
  if (zlo >= zhi) return;
  const int group = n_heads / n_kv_heads;
  const int kvd = n_kv_heads * hd;
  const int r4 = hd / 4, nf4 = ATTN_CHUNK * r4;
  const int gh = group * hd;
  const float scale = 1.0f / sqrtf(static_cast<float>(hd));
  const size_t head_off = static_cast<size_t>(kvh) * hd;

  AttnRegs<NV> R;
  attn_load_chunk<NV>(R, kc, vc, c, pos0 + zhi, kvd, head_off, r4, nf4);
  // the queries of tokens z .. z+NT-1 (tokens past the tile re-read its last)
  auto load_q = [&](int z, float (&qv)[NT][NQ]) {
#pragma unroll
    for (int k = 0; k < NT; ++k) {
      const float* qg = q + static_cast<size_t>(min(z + k, zhi - 1)) * tok_q + static_cast<size_t>(kvh) * gh;
#pragma unroll
      for (int u = 0; u < NQ; ++u) qv[k][u] = qg[min(tid + 256 * u, gh - 1)];
    }
  };
  float qv[NT][NQ];
  load_q(zlo, qv);
#pragma unroll
  for (int u = 0; u < NV; ++u) {
    const int f = min(tid + 256 * u, nf4 - 1);
    const int j = f / r4, c4 = f - j * r4;
    *reinterpret_cast<f32x4*>(&sK[j * KS + (SWZ ? (c4 ^ (j & 15)) : c4) * 4]) = R.k[u];
    *reinterpret_cast<f32x4*>(&sV[j * HDM + c4 * 4]) = R.v[u];
  }
  if constexpr (WL) __syncthreads();  // the staged rows
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int z = zlo; z < zhi; z += NT) {
    // the previous tokens' readers of sQ, sE and sMZ are done (and, first, the
    // staged rows are in)
    if constexpr (WL) wave_sync();
    else __syncthreads();
#pragma unroll
    for (int k = 0; k < NT; ++k) {
#pragma unroll
      for (int u = 0; u < NQ; ++u) {
        const int i = tid + 256 * u;
        if (i < gh) sQ[k * QSZ + (i / hd) * HDM + i % hd] = qv[k][u];
      }
    }
    if (z + NT < zhi) load_q(z + NT, qv);
    if constexpr (WL) wave_sync();
    else __syncthreads();
    int Tk[NT];
#pragma unroll
    for (int k = 0; k < NT; ++k) Tk[k] = pos0 + min(z + k, zhi - 1) + 1;
    float o[NT][OPT];
    auto put_mz = [&](int k, int hh, float2 v) {
      if constexpr (SWZ) {
        if (z + k < zhi)
          part_mz[static_cast<size_t>(z + k) * tok_mz + static_cast<size_t>(kvh * group + hh) * max_chunks + c] = v;
      } else {
        sMZ[k * ATTN_MAX_GROUP + hh] = v;
      }
    };
    attn_tokens_chunk<HDM, OPT, NT, WL, GM, SWZ>(sK, sV, sQ, sE, put_mz, c, Tk, group, hd, gh, scale, o);
#pragma unroll
    for (int k = 0; k < NT; ++k) {
      if (z + k < zhi) {
        float* po = part_o + static_cast<size_t>(z + k) * tok_o;
#pragma unroll
        for (int u = 0; u < OPT; ++u) {
          const int oi = tid + 256 * u;
          if (oi < gh) {
            const int hh = oi / hd, i = oi - hh * hd;
            po[(static_cast<size_t>(kvh * group + hh) * max_chunks + c) * hd + i] = o[k][u];
          }
        }
        if constexpr (SWZ) {
          // stored by put_mz
        } else if constexpr (WL) {
          // lane 0 of the wave that wrote them: heads wave, wave + 4
          for (int hh = wave; hh < group; hh += 4)
            if (lane == 0)
              part_mz[static_cast<size_t>(z + k) * tok_mz + static_cast<size_t>(kvh * group + hh) * max_chunks + c] =
                  sMZ[k * ATTN_MAX_GROUP + hh];
        } else if (tid < group) {
          part_mz[static_cast<size_t>(z + k) * tok_mz + static_cast<size_t>(kvh * group + tid) * max_chunks + c] =
              sMZ[k * ATTN_MAX_GROUP + tid];
        }
      }
    }
  }
}

// The combine over a head's chunks for output i (head h, dim d), in chunk
// order: m = max m_c; f_c = exp(m_c - m); Z = fma(z_c, f_c, Z);
// O = fma(o_c[d], f_c, O); out = O / Z.
__global__ void k_attn_combine(const float* __restrict__ part_o, const float2* __restrict__ part_mz,
                               const int* __restrict__ state, int n_out, int hd, int max_chunks,
                               float* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_out) return;
  const int nch = state[1] / ATTN_CHUNK + 1;
  const int h = i / hd, d = i - h * hd;
  const float2* mz = part_mz + static_cast<size_t>(h) * max_chunks;
  const float* o = part_o + static_cast<size_t>(h) * max_chunks * hd + d;
  float m = mz[0].x;
  for (int c = 1; c < nch; ++c) m = fmaxf(m, mz[c].x);
  float Z = 0.0f, O = 0.0f;
  for (int c = 0; c < nch; ++c) {
    const float f = exp_f32(mz[c].x - m);
    Z = __builtin_fmaf(mz[c].y, f, Z);
    O = __builtin_fmaf(o[static_cast<size_t>(c) * hd], f, O);
  }
  out[i] = O / Z;
}

hipError_t launch_attention(const float* q, const float* kc, const float* vc, const int* state, int n_heads,
                            int n_kv_heads, int head_dim, int max_chunks, const AttnPart& part, hipStream_t s) {
  if (head_dim <= 0 || head_dim > 128 || head_dim % 4 || n_heads % n_kv_heads ||
      n_heads / n_kv_heads > ATTN_MAX_GROUP)
    return hipErrorInvalidValue;
  const dim3 grid(n_kv_heads, attn_max_splits(1, max_chunks));
  if (head_dim <= 64)
    launch_kernel(head_dim == 64 ? k_attention<64, true> : k_attention<64, false>, grid, dim3(256), 0, s, q, kc, vc,
                  state, n_heads, n_kv_heads, head_dim,
                  max_chunks, part.o, part.mz, -1, size_t{0}, size_t{0}, size_t{0});
  else
    launch_kernel(k_attention<128, false>, grid, dim3(256), 0, s, q, kc, vc, state, n_heads, n_kv_heads, head_dim,
                  max_chunks, part.o, part.mz, -1, size_t{0}, size_t{0}, size_t{0});
  return hipGetLastError();
}

hipError_t launch_attention_q8k(const float* q, const float* kc, const float* vc, const int* state, int n_heads,
                                int n_kv_heads, int head_dim, BlockQ8K* out, unsigned* err, hipStream_t s) {
  if (!attn_q8k_fits(n_heads, n_kv_heads, head_dim)) return hipErrorInvalidValue;
  launch_kernel(k_attention_q8k, dim3(n_kv_heads), dim3(256 * AQ_GROUPS), 0, s, q, kc, vc, state, n_heads, n_kv_heads,
                out, err);
  return hipGetLastError();
}

hipError_t launch_attention_batch(const float* q, const float* kc, const float* vc, int n_heads, int n_kv_heads,
                                  int head_dim, int max_chunks, const AttnPart& part, size_t tok_o, size_t tok_mz,
                                  int pos0, int n_tok, hipStream_t s) {
  if (head_dim <= 0 || head_dim > 128 || head_dim % 4 || n_heads % n_kv_heads ||
      n_heads / n_kv_heads > ATTN_MAX_GROUP || pos0 < 0)
    return hipErrorInvalidValue;
  if (n_tok <= 0) return hipSuccess;
  // one work group per (kv head, chunk, token tile); tiles whose tokens do
  // not reach a chunk return at once
  // tokens per tile (MCPM_PREFILL_ATTN_TT overrides, a tuning aid)
  static const int tt_env = [] {
    const char* v = std::getenv("MCPM_PREFILL_ATTN_TT");
    return v ? std::atoi(v) : 0;
  }();
  const int tt = tt_env >= 1 && tt_env <= 256 ? tt_env : 16;
  const dim3 grid(n_kv_heads, (pos0 + n_tok - 1) / ATTN_CHUNK + 1, (n_tok + tt - 1) / tt);
  const size_t tok_q = static_cast<size_t>(n_heads) * head_dim;
  if (head_dim == 64 && n_heads / n_kv_heads <= 4)
    hipLaunchKernelGGL((k_attention_tile<64, true, 4>), grid, dim3(256), 0, s, q, kc, vc, n_heads, n_kv_heads,
                       head_dim, max_chunks, part.o, part.mz, pos0, n_tok, tt, tok_q, tok_o, tok_mz);
  else if (head_dim == 64)
    hipLaunchKernelGGL((k_attention_tile<64, true, 8>), grid, dim3(256), 0, s, q, kc, vc, n_heads, n_kv_heads, head_dim,
                       max_chunks, part.o, part.mz, pos0, n_tok, tt, tok_q, tok_o, tok_mz);
  else if (head_dim < 64)
    hipLaunchKernelGGL((k_attention_tile<64, false, 8>), grid, dim3(256), 0, s, q, kc, vc, n_heads, n_kv_heads, head_dim,
                       max_chunks, part.o, part.mz, pos0, n_tok, tt, tok_q, tok_o, tok_mz);
  else
    hipLaunchKernelGGL((k_attention_tile<128, false, 8>), grid, dim3(256), 0, s, q, kc, vc, n_heads, n_kv_heads, head_dim,
                       max_chunks, part.o, part.mz, pos0, n_tok, tt, tok_q, tok_o, tok_mz);
  return hipGetLastError();
}

hipError_t launch_attn_combine(const AttnPart& part, const int* state, int n_heads, int head_dim, int max_chunks,
                               float* out, hipStream_t s) {
  const int n = n_heads * head_dim;
  hipLaunchKernelGGL(k_attn_combine, dim3((n + 255) / 256), dim3(256), 0, s, part.o, part.mz, state, n, head_dim,
                     max_chunks, out);
  return hipGetLastError();
}

__global__ void k_dequant_rows(const WView w, int row0, int n_rows, int cols, float* __restrict__ out) {
  const int r = row0 + blockIdx.y;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < cols; i += gridDim.x * blockDim.x) {
    float v;
    if (w.type == MCPM_TYPE_Q8_0) {
      const size_t blk = static_cast<size_t>(i / QK8_0) * w.rows + r;
      const int8_t q = static_cast<int8_t>(w.p0[blk * 32 + i % QK8_0]);
      const uint16_t dh = w.p1[blk * 2] | (w.p1[blk * 2 + 1] << 8);
      v = fp16_to_fp32(dh) * static_cast<float>(q);
    } else if (w.type == MCPM_TYPE_F32) {
      v = reinterpret_cast<const float*>(w.p0)[static_cast<size_t>(r) * cols + i];
    } else {
      v = dequant_value(w, r, i / QK_K, i % QK_K);
    }
    out[static_cast<size_t>(blockIdx.y) * cols + i] = v;
  }
}

hipError_t launch_dequant_rows(const WView& w, int row0, int n_rows, int cols, float* out, hipStream_t s) {
  hipLaunchKernelGGL(k_dequant_rows, dim3((cols + 255) / 256, n_rows), dim3(256), 0, s, w, row0, n_rows, cols, out);
  return hipGetLastError();
}

// get_embedding: row `token` (from the step state) dequantized to x; one
// work group per 256-value block, one value per thread.  epoch (optional):
// advanced by one, by one thread.
__global__ void __launch_bounds__(256) k_embedding(const WView w, const int* __restrict__ state, int dim,
                                                   float* __restrict__ out, unsigned* epoch) {
  const int token = state[0];
  const int i = blockIdx.x * QK_K + threadIdx.x;
  if (i < dim) out[i] = dequant_value(w, token, blockIdx.x, threadIdx.x);
  if (epoch && i == 0) epoch[0] = epoch[0] + 1u;
}

hipError_t launch_embedding(const WView& w, const int* state, int dim, float* out, hipStream_t s,
                            unsigned* epoch) {
  hipLaunchKernelGGL(k_embedding, dim3((dim + QK_K - 1) / QK_K), dim3(QK_K), 0, s, w, state, dim, out, epoch);
  return hipGetLastError();
}

// ------------------------------------------------- fp32-activation GEMVs ----
// gemv_f32 (src/ops/ops.cpp:32-43): lane t sums w*x over c = t, t+64, ...
// (multiply then add), then the 64-lane pairwise tree.  One wave per row.
__global__ void __launch_bounds__(256) k_gemv_f32(const float* __restrict__ w, const float* __restrict__ x,
                                                  float* __restrict__ out, int rows, int cols) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (r >= rows) return;
  const float* wr = w + static_cast<size_t>(r) * cols;
  float p = 0.0f;
  for (int c = lane; c < cols; c += 64) p = p + wr[c] * x[c];
  p = wave_tree_sum(p);
  if (lane == 0) out[r] = p;
}

hipError_t launch_gemv_f32(const float* w, const float* x, float* out, int rows, int cols, hipStream_t s) {
  hipLaunchKernelGGL(k_gemv_f32, dim3((rows + 3) / 4), dim3(256), 0, s, w, x, out, rows, cols);
  return hipGetLastError();
}

// Read-only pass: every 16-byte word of src once (non-temporal loads, as the
// GEMVs stream their weights), a grid-stride loop over `grid` work groups; one
// xor per work group goes to out so the loads stay.  Its duration is the floor
// of one launch that reads as many bytes as a GEMV class.
__global__ void __launch_bounds__(256) k_stream_read(const u32x4* __restrict__ src, size_t n16,
                                                     uint32_t* __restrict__ out) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  uint32_t acc = 0;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride) {
    const u32x4 v = __builtin_nontemporal_load(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  __shared__ uint32_t s[256];
  s[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t a = 0;
    for (int t = 0; t < 256; ++t) a ^= s[t];
    out[blockIdx.x] = a;
  }
}

hipError_t launch_stream_read(const void* src, size_t bytes, int grid, uint32_t* out, hipStream_t s) {
  launch_kernel(k_stream_read, dim3(grid), dim3(256), 0, s, static_cast<const u32x4*>(src), bytes / 16, out);
  return hipGetLastError();
}

// gemv_q8_0 (src/ops/ops.cpp:58-79): per block s = sum over i of float(q_i)*x_i
// (i ascending, multiply then add); row = row + s*d over blocks in order.
// One lane per row.
__global__ void __launch_bounds__(256) k_gemv_q8_0(const WView w, const float* __restrict__ x,
                                                   float* __restrict__ out, int rows, int cols) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int nb = cols / QK8_0;
  float row = 0.0f;
  for (int b = 0; b < nb; ++b) {
    const size_t blk = static_cast<size_t>(b) * w.rows + r;
    const int8_t* q = reinterpret_cast<const int8_t*>(w.p0 + blk * 32);
    float s = 0.0f;
    for (int i = 0; i < QK8_0; ++i) s = s + static_cast<float>(q[i]) * x[b * QK8_0 + i];
    const uint16_t dh = w.p1[blk * 2] | (w.p1[blk * 2 + 1] << 8);
    row = row + s * fp16_to_fp32(dh);
  }
  out[r] = row;
}

hipError_t launch_gemv_q8_0(const WView& w, const float* x, float* out, int rows, int cols, hipStream_t s) {
  hipLaunchKernelGGL(k_gemv_q8_0, dim3((rows + 255) / 256), dim3(256), 0, s, w, x, out, rows, cols);
  return hipGetLastError();
}

// ------------------------------------------------------------- argmax ------
__global__ void __launch_bounds__(256) k_argmax_partial(const float* __restrict__ x, int n, float2* __restrict__ part) {
  __shared__ float sv[4];
  __shared__ int si[4];
  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
    const float v = x[i];
    if (v > bv || (v == bv && i < bi)) {
      bv = v;
      bi = i;
    }
  }
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < 4; ++k)
      if (sv[k] > bv || (sv[k] == bv && si[k] < bi)) {
        bv = sv[k];
        bi = si[k];
      }
    part[blockIdx.x] = make_float2(bv, __int_as_float(bi));
  }
}

hipError_t launch_argmax_partial(const float* x, int n, float2* part, int nparts, hipStream_t s) {
  hipLaunchKernelGGL(k_argmax_partial, dim3(nparts), dim3(256), 0, s, x, n, part);
  return hipGetLastError();
}

// Reduces (value, index) partials to the first index of the maximum; writes
// it to out_token, and when a step state is given, feeds it back as the next
// input token, appends it to out_tokens and advances pos.
// Final argmax over the partials (value, index) of the LM-head work groups:
// the largest value, ties to the lowest index.  256 threads, loads issued 16
// at a time; slots past nparts re-read the last partial (harmless for a max).
__global__ void __launch_bounds__(256) k_argmax_final(const float2* __restrict__ part, int nparts,
                                                      int* __restrict__ out_token, StepState* st,
                                                      int* __restrict__ out_tokens) {
  __shared__ float s_v[4];
  __shared__ int s_i[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
  for (int i0 = tid; i0 < nparts; i0 += 256 * 16) {
    float2 v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = part[min(i0 + 256 * k, nparts - 1)];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const float pv = v[k].x;
      const int pi = __float_as_int(v[k].y);
      if (pv > bv || (pv == bv && pi < bi)) {
        bv = pv;
        bi = pi;
      }
    }
  }
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    s_v[wave] = bv;
    s_i[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w) {
      if (s_v[w] > bv || (s_v[w] == bv && s_i[w] < bi)) {
        bv = s_v[w];
        bi = s_i[w];
      }
    }
    if (out_token) *out_token = bi;
    if (st) {
      st->token = bi;
      st->pos = st->pos + 1;
      if (out_tokens && st->step < st->n_out) out_tokens[st->step] = bi;
      st->step = st->step + 1;
    }
  }
}

hipError_t launch_argmax_final(const float2* part, int nparts, int* out_token, StepState* st, int* out_tokens,
                               hipStream_t s) {
  hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, s, part, nparts, out_token, st, out_tokens);
  return hipGetLastError();
}

__global__ void k_fill_f32(float* p, float v, size_t n) {
  const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

hipError_t launch_fill_f32(float* p, float v, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill_f32, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, p, v, n);
  return hipGetLastError();
}

}  // namespace mcpm
