// mcpm_gemv.hip -- the Q4_K / Q6_K x Q8_K GEMV family (QKV, O, gate/up, down,
// LM head and the per-op entry points).
//
// Arithmetic.  A row dot is that of one AVX2 row (src/ops/ops_avx2.cpp:153-196
// for Q4_K, 201-276 for Q6_K): per block, eight integer lane sums isum[m]
// (lane m owns bytes 4m..4m+3 of every 32-byte chunk), then, blocks in order,
//   acc[m] = fma(d_x*d_w, float(isum[m]), acc[m])
//   Q4_K:  acc_min = fma(-(d_x*dmin_w), float(minsum), acc_min)
//   row = ((acc0+acc4)+(acc2+acc6)) + ((acc1+acc5)+(acc3+acc7))  [+ acc_min]
// Integer sums are exact, so how they are formed is free; the float chain is
// the reference's.
//
// Work.  One GPU lane forms all eight isum of one (row, block) from the
// block's bytes (a 16-byte load per chunk, consecutive lanes on consecutive
// rows) and the Q8_K activations in LDS.  Two shapes:
//   ROW   a lane owns one row, visits its blocks in order and keeps the float
//         chain in registers; a wave covers 64 rows.
//   TILE  a wave covers S rows ("slots") of all nb blocks: pair q = lane +
//         64k (k < KB steps) is block q / S of slot q % S.  The lanes leave
//         (isum[8], d_x*d_w, d_x*dmin_w, minsum) per (block, slot) in LDS,
//         then 4 lanes per row run the chain over the blocks in order.
// Each wave streams its (item, step) sequence through two register sets,
// loading one step ahead.  Loads are unconditional within a path: rows and
// blocks past the end are clamped into the tensor and their results masked;
// waves of one or two steps load no step past their last.
// Work groups share the activations (prologue) and nothing else.
#include <algorithm>
#include <cstdlib>
#include <cstdio>
#include <cstring>

#include "mcpm_attn.h"
#include "mcpm_device.h"

namespace mcpm {

typedef short i16x2 __attribute__((ext_vector_type(2)));

// A copy of a wave-uniform value in a scalar register, so the compiler knows
// it is uniform across the wave.
__device__ __forceinline__ int sgpr(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Region reg's copy of a field, selected by value: a ?: over two lvalues is an
// lvalue, i.e. a select of addresses and one load through it.
template <typename T>
__device__ __forceinline__ T pick(int reg, T a, T b, T c) {
  return reg == 2 ? c : reg == 1 ? b : a;
}
#define MCPM_PICK(reg, A, B, C, f) pick((reg), (A).f, (B).f, (C).f)

// ------------------------------------------------------------- LDS plan ----
// Dynamic LDS in dwords, by blocks per row nb:
//   xs   [nb][68]  Q8_K quants of block b (64 dwords, native order) + pad
//   xd   [nb]      Q8_K d
//   xbp  [nb][4]   (bsums[4i]+bsums[4i+1], bsums[4i+2]+bsums[4i+3]) as i16 pairs
//   xbs  [nb][16]  bsums as ints
//   red  [260]     reduction scratch
//   vrow [NW][64]  TILE: row values of each wave's current item
//   U              PRO_ATTN_EVEN / PRO_ATTN_ONE: the fp32 attention output
//                  (nb*256), later the TILE chain areas (NW waves x nb*S*12)
//   at             PRO_ATTN_ONE: the staged chunk of one kv head (AttnLds)
// Every region starts on a 16-byte boundary.
struct LdsPlan {
  int xs, xd, xbp, xbs, red, vrow, u, at, words;
};

// attn: 0 none, 1 PRO_ATTN_EVEN, 2 PRO_ATTN_ONE
__host__ __device__ inline LdsPlan lds_plan(int nb, int S, bool tile, int attn, int NW) {
  LdsPlan L;
  L.xs = 0;
  L.xd = nb * 68;
  L.xbp = L.xd + ((nb + 3) & ~3);
  L.xbs = L.xbp + nb * 4;
  L.red = L.xbs + nb * 16;
  L.vrow = L.red + 260;
  L.u = L.vrow + (tile ? NW * 64 : 0);
  const int usz = tile ? NW * nb * S * 12 : 0;
  L.words = L.u + (attn && nb * QK_K > usz ? nb * QK_K : usz);
  L.at = L.words;
  if (attn == 2) L.words += static_cast<int>((AttnLds<64>::bytes + 15) / 16 * 4);
  return L;
}

template <int PRO>
constexpr int lds_attn() {
  return PRO == PRO_ATTN_EVEN ? 1 : PRO == PRO_ATTN_ONE ? 2 : 0;
}

// ------------------------------------------------------------- prologue ----
// Each row of 16 lanes takes one block: block 4*NW*r + 4*wave + row (round r,
// row = lane/16, NW >= 4 waves), lane j = lane%16 holding values 16j..16j+15
// (one Q8_K bsum group).  Blocks past nb re-read block nb-1 (in bounds,
// results unused).
constexpr int NR = (MAX_NB + 15) / 16;
constexpr int CHAIN_BATCH = 12;  // TILE chain: blocks whose LDS entries are read together

// PRO_ATTN_EVEN: thread t < 32*nb combines the ATTN_VALS values t*8 .. t*8+7
// (one head: head_dim % 8 == 0, nb <= 8) over the chunks.  The o_c of the
// first ATTN_RB chunks and the (m_c, z_c) of the first ATTN_MZ are loaded with
// the activations, before the weights; further chunks' partials (and their
// maxima) follow in batches of ATTN_BATCH, a batch's loads issued together.
// Larger batches or preloads cost more than they save: their registers push
// the kernel past 256 VGPRs into AGPR copies, which slows short contexts.
constexpr int ATTN_VALS = 8, ATTN_RB = 4, ATTN_MZ = 8, ATTN_BATCH = 8, ATTN_MAX_NB = 8;

struct ProRegs {
  f32x4 x[NR][4];  // fp32 activations of the lane's 16 values
  f32x4 g[NR][4];  // RMSNorm weights, same layout
  float xp[MAX_NB];  // RMSNorm: x[t], x[t+256], ... of thread t < 256 (its partial's terms)
  f32x4 ao[ATTN_RB][2];  // PRO_ATTN_EVEN: o_c of thread t's 8 values, chunks 0..ATTN_RB-1
  float2 amz[ATTN_MZ];   // (m_c, z_c) of its head, chunks 0..ATTN_MZ-1
  AttnRegs<4> kv;        // PRO_ATTN_ONE: the chunk's K and V rows of the work group's kv head
  f32x4 aq;              // and a float4 of its query heads
  u32x4 q[NR];     // Q8_K codes of the lane's 16 values
  int bs[NR];      // Q8_K bsums[j]
  float d[NR];     // Q8_K d
};

// Coherence of a GEMV phase's accesses to data other work groups of the same
// launch write or read (the fused kernels), a bitmask: COH_IN the
// activations, COH_OUT the epilogue outputs.  Other data (written by earlier
// launches, or read and written by the same lane) takes plain accesses.
constexpr int COH_IN = 1, COH_OUT = 2;

template <int PRO, int COH = 0>
__device__ __forceinline__ void prologue_load(const GemvArgs& a, int NW, int wave, int lane, ProRegs& X) {
  static_assert(!((COH & COH_IN) && PRO == PRO_ATTN_EVEN), "coherent partial reads are not implemented");
  constexpr bool cin = (COH & COH_IN) != 0;
  const int nb = a.nb, row = lane >> 4, j = lane & 15;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    if (4 * NW * r + 4 * wave < nb) {  // uniform in the wave: waves past the blocks skip
      const int b = min(4 * NW * r + 4 * wave + row, nb - 1);
      if constexpr (PRO == PRO_ATTN_EVEN || PRO == PRO_ATTN_ONE) {
        // the activations are formed in LDS by prologue_compute
      } else if constexpr (PRO == PRO_Q8K) {
        const BlockQ8K* blk = a.xq + b;
        const uint32_t* q = reinterpret_cast<const uint32_t*>(blk->qs) + 4 * j;  // 4-byte aligned only
        X.q[r] = u32x4{q[0], q[1], q[2], q[3]};
        X.bs[r] = blk->bsums[j];
        X.d[r] = blk->d;
      } else {
        const f32x4* xp = reinterpret_cast<const f32x4*>(a.x + b * QK_K + 16 * j);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (cin) X.x[r][i] = ld_coh4(a.x, static_cast<uint32_t>((b * QK_K + 16 * j + 4 * i) * 4));
          else X.x[r][i] = xp[i];
        }
        if constexpr (PRO == PRO_NORM_AWAY || PRO == PRO_NORM_EVEN) {
          const f32x4* gp = reinterpret_cast<const f32x4*>(a.gamma + b * QK_K + 16 * j);
#pragma unroll
          for (int i = 0; i < 4; ++i) X.g[r][i] = gp[i];
        }
      }
    }
  }
  if constexpr (PRO == PRO_ATTN_ONE) {
    // this work group's kv head's chunk and query heads (attn_xcd_heads), issued
    // before the weights
    const int t = static_cast<int>(threadIdx.x), jw = static_cast<int>(blockIdx.x) / 8, hpw = a.attn_hpw;
    const int h0 = jw * hpw;
    if (h0 < nb * QK_K / 64) {
      attn_load_chunk<4>(X.kv, a.k_cache, a.v_cache, 0, a.state[1] + 1, a.kvd, static_cast<size_t>(h0 / 4) * 64,
                         16, ATTN_CHUNK * 16);
      if (t < hpw * 16) X.aq = reinterpret_cast<const f32x4*>(a.x + static_cast<size_t>(h0) * 64)[t];
    }
  }
  if constexpr (PRO == PRO_ATTN_EVEN) {
    const int t = static_cast<int>(threadIdx.x);
    if (t * ATTN_VALS >= nb * QK_K) return;  // threads 0..32*nb-1 form the activations
    const int hd = a.head_dim, maxc = a.attn_max_chunks;
    const int i0 = t * ATTN_VALS, h = i0 / hd, d0 = i0 - h * hd;
    const int last = a.state[1] / ATTN_CHUNK;  // chunks 0..last
    const float2* mz = a.attn_mz + static_cast<size_t>(h) * maxc;
    // only the chunks present (uniform branches)
#pragma unroll
    for (int c = 0; c < ATTN_MZ; ++c)
      if (c <= last) X.amz[c] = mz[c];
#pragma unroll
    for (int c = 0; c < ATTN_RB; ++c) {
      if (c <= last) {
        const f32x4* o = reinterpret_cast<const f32x4*>(a.x + (static_cast<size_t>(h) * maxc + c) * hd + d0);
        X.ao[c][0] = o[0];
        X.ao[c][1] = o[1];
      }
    }
  }
  if constexpr (PRO == PRO_NORM_AWAY || PRO == PRO_NORM_EVEN) {
    if (wave >= 4) return;  // threads 0..255 hold the RMS partials
    const int t = static_cast<int>(threadIdx.x);
#pragma unroll
    for (int g = 0; g < MAX_NB / 8; ++g) {
      if (8 * g < nb) {  // uniform
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float* xv = a.x + min(8 * g + k, nb - 1) * QK_K + t;
          X.xp[8 * g + k] = cin ? ld_coh(xv) : *xv;
        }
      }
    }
  }
}

// Block b (lane j of its row) into LDS: codes, d, bsums and the bsum pair
// sums.  Every lane of the row takes part (lane moves); `live` gates stores.
__device__ __forceinline__ void store_xblock(uint32_t* L, const LdsPlan& P, int b, int j, bool live, u32x4 q,
                                             float d, int bs) {
  // bsums[2g] + bsums[2g+1] on lane 2g; pairs (2i, 2i+1) on lane 4i
  const int v = bs + dpp_i<DPP_XOR1>(bs);
  const uint32_t w = (static_cast<uint32_t>(v) & 0xffffu) | (static_cast<uint32_t>(dpp_i<DPP_XOR2>(v)) << 16);
  if (live) {
    *reinterpret_cast<u32x4*>(L + P.xs + b * 68 + 4 * j) = q;
    L[P.xbs + b * 16 + j] = static_cast<uint32_t>(bs);
    if (j == 0) L[P.xd + b] = __float_as_uint(d);
    if ((j & 3) == 0) L[P.xbp + b * 4 + (j >> 2)] = w;
  }
}

// PRO_ATTN_EVEN: the attention output x[i] of threads' values (head h, dim
// d) from the chunk partials, in chunk order (k_attn_combine's arithmetic):
// m = max m_c; f_c = exp(m_c - m); Z = fma(z_c, f_c, Z); O = fma(o_c[d], f_c, O);
// x = O / Z, into sx (fp32, nb*256).
__device__ __forceinline__ void attn_combine_values(const GemvArgs& a, const ProRegs& X, float* sx) {
  const int hd = a.head_dim, maxc = a.attn_max_chunks;
  const int t = static_cast<int>(threadIdx.x);
  const int i0 = t * ATTN_VALS, h = i0 / hd, d0 = i0 - h * hd;
  const int nch = a.state[1] / ATTN_CHUNK + 1;
  const float2* mzp = a.attn_mz + static_cast<size_t>(h) * maxc;
  const float* op = a.x + static_cast<size_t>(h) * maxc * hd + d0;
  // When the context has them: chunks ATTN_RB .. ATTN_RB+ATTN_BATCH-1 and the
  // maxima of chunks ATTN_MZ .. ATTN_MZ+ATTN_BATCH-1, all issued together at
  // indices clamped to the last chunk (a repeated maximum changes nothing;
  // repeated o_c are not used), the maxima first.
  const bool more_mz = nch > ATTN_MZ, more_o = nch > ATTN_RB;  // uniform
  float mb[ATTN_BATCH];
  if (more_mz) {
#pragma unroll
    for (int k = 0; k < ATTN_BATCH; ++k) mb[k] = mzp[min(ATTN_MZ + k, nch - 1)].x;
  }
  f32x4 ob[ATTN_BATCH][2];
  float2 zb[ATTN_BATCH];
  auto load_batch = [&](int c0) {
#pragma unroll
    for (int k = 0; k < ATTN_BATCH; ++k) {
      const int c = min(c0 + k, nch - 1);
      zb[k] = mzp[c];
      const f32x4* o = reinterpret_cast<const f32x4*>(op + static_cast<size_t>(c) * hd);
      ob[k][0] = o[0];
      ob[k][1] = o[1];
    }
  };
  if (more_o) load_batch(ATTN_RB);
  float m = X.amz[0].x;
#pragma unroll
  for (int c = 1; c < ATTN_MZ; ++c)
    if (c < nch) m = fmaxf(m, X.amz[c].x);
  if (more_mz) {
#pragma unroll
    for (int k = 0; k < ATTN_BATCH; ++k) m = fmaxf(m, mb[k]);
  }
  for (int c0 = ATTN_MZ + ATTN_BATCH; c0 < nch; c0 += ATTN_BATCH) {
#pragma unroll
    for (int k = 0; k < ATTN_BATCH; ++k) mb[k] = mzp[min(c0 + k, nch - 1)].x;
#pragma unroll
    for (int k = 0; k < ATTN_BATCH; ++k) m = fmaxf(m, mb[k]);
  }
  float Z = 0.0f;
  f32x4 O[2] = {f32x4{0.0f, 0.0f, 0.0f, 0.0f}, f32x4{0.0f, 0.0f, 0.0f, 0.0f}};
  auto step = [&](float2 mz, const f32x4 (&o)[2]) {
    const float f = exp_f32(mz.x - m);
    Z = __builtin_fmaf(mz.y, f, Z);
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      O[v].x = __builtin_fmaf(o[v].x, f, O[v].x);
      O[v].y = __builtin_fmaf(o[v].y, f, O[v].y);
      O[v].z = __builtin_fmaf(o[v].z, f, O[v].z);
      O[v].w = __builtin_fmaf(o[v].w, f, O[v].w);
    }
  };
  // the steps in chunk order
#pragma unroll
  for (int c = 0; c < ATTN_RB; ++c)
    if (c < nch) step(X.amz[c], X.ao[c]);
  for (int c0 = ATTN_RB; c0 < nch; c0 += ATTN_BATCH) {
    if (c0 > ATTN_RB) load_batch(c0);
#pragma unroll
    for (int k = 0; k < ATTN_BATCH; ++k)
      if (c0 + k < nch) step(zb[k], ob[k]);
  }
#pragma unroll
  for (int v = 0; v < 2; ++v) {
    const f32x4 r = O[v];
    *reinterpret_cast<f32x4*>(sx + i0 + 4 * v) = f32x4{r.x / Z, r.y / Z, r.z / Z, r.w / Z};
  }
}

// attn_combine_values on the threads that hold values, then a work-group
// barrier.
__device__ __forceinline__ void attn_combine(const GemvArgs& a, const ProRegs& X, float* sx) {
  // threads past the values take no part but the barrier, which every thread
  // reaches exactly once (a wave may hold both kinds when nb == 1)
  if (static_cast<int>(threadIdx.x) * ATTN_VALS < a.nb * QK_K) attn_combine_values(a, X, sx);
  __syncthreads();
}

// PRO_ATTN_ONE: the attention output of every head over a context of
// T = pos + 1 <= 64 positions (one chunk), into sx (src/ops/ops.cpp:537-628,
// the oracle's or_attention), shared among the work groups of each XCD:
// work group b runs on XCD x = b % 8 and is the j = b / 8-th there; for
// j*hpw < heads it computes query heads h0 = j*hpw .. h0+hpw-1 (one kv
// head's) with attn_token_chunk on the chunk's K and V rows (R, loaded by
// prologue_load ahead of the weights) and its queries (q) staged in LDS,
// then the one-chunk combine x = fma(o, f, 0) / fma(z_c, f, 0),
// f = exp(m_c - m), m = m_c, and stores each value as a (value, tag) record
// in XCD x's array at workgroup scope: the vector L1 writes through and the
// line stays in that XCD's L2.  Every work group then waits for all records
// of its XCD (agent-scope loads, which miss the L1 and find them in the
// L2), at most spin_limit polls; past it, or on a work group that does not
// run on the XCD recorded at set-up, the error word is set and the values
// are not used.  All work groups of the launch must be resident (grid <=
// CUs).  Needs 256 threads; ends with a barrier.
__device__ __forceinline__ void attn_xcd_heads(const GemvArgs& a, const AttnRegs<4>& R, f32x4 q, float* sx,
                                               float* scratch) {
  constexpr int HD = 64;
  const int t = static_cast<int>(threadIdx.x), b = static_cast<int>(blockIdx.x);
  const int x = b % 8, jw = b / 8, T = a.state[1] + 1, nh = a.nb * QK_K / HD, hpw = a.attn_hpw;
  const uint32_t tag = a.epoch[0] * a.tag_mul + a.tag_add;
  uint64_t* rec = a.xrec + static_cast<size_t>(x) * nh * HD;
  bool bad = static_cast<int>(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15u) != a.xcc[x];  // XCC_ID, bits 3:0
  if (jw * hpw < nh && !bad) {
    const int h0 = jw * hpw;
    const AttnLds<HD> A(scratch);
    if (t < hpw * (HD / 4)) reinterpret_cast<f32x4*>(A.sQ)[t] = q;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int f = t + 256 * u, jr = f >> 4, c4 = f & 15;
      *reinterpret_cast<f32x4*>(&A.sK[jr * (HD + 4) + c4 * 4]) = R.k[u];
      *reinterpret_cast<f32x4*>(&A.sV[jr * HD + c4 * 4]) = R.v[u];
    }
    __syncthreads();
    float o[1];
    attn_token_chunk<HD, 1>(A.sK, A.sV, A.sQ, A.sE, A.sMZ, 0, T, hpw, HD, hpw * HD,
                            1.0f / sqrtf(static_cast<float>(HD)), o, t);
    if (t < hpw * HD) {
      const float2 mz = A.sMZ[t / HD];
      const float f = exp_f32(mz.x - mz.x);  // one chunk: m = m_c
      const float v = __builtin_fmaf(o[0], f, 0.0f) / __builtin_fmaf(mz.y, f, 0.0f);
      __hip_atomic_store(rec + h0 * HD + t, (static_cast<uint64_t>(tag) << 32) | __float_as_uint(v),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
  // every record of the XCD: thread t's records t + 256k
  constexpr int KR = ATTN_MAX_NB;  // nh*64 = nb*256 <= 2048
  uint64_t r[KR];
#pragma unroll
  for (int k = 0; k < KR; ++k) {
    const int i = t + 256 * k;
    r[k] = i < nh * HD && !bad ? __hip_atomic_load(rec + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                               : static_cast<uint64_t>(tag) << 32;
  }
  for (unsigned spins = 0;; ++spins) {
    unsigned pend = 0;
#pragma unroll
    for (int k = 0; k < KR; ++k)
      if (static_cast<uint32_t>(r[k] >> 32) != tag) pend |= 1u << k;
    if (!pend) break;
    if (spins >= a.spin_limit) {
      bad = true;
      break;
    }
#pragma unroll
    for (int k = 0; k < KR; ++k)
      if (pend >> k & 1u) r[k] = __hip_atomic_load(rec + t + 256 * k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (bad) __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
  for (int k = 0; k < KR; ++k) {
    const int i = t + 256 * k;
    if (i < nh * HD) sx[i] = __uint_as_float(static_cast<uint32_t>(r[k]));
  }
  __syncthreads();
}

// Q8_K activations of the work group into LDS: as given (PRO_Q8K), or
// quantized from fp32 (ties-even or ties-away), optionally after RMSNorm
// (src/ops/ops.cpp:676-723, 745-789).  Ends with a work-group barrier.
template <int PRO>
__device__ __forceinline__ void prologue_compute(const GemvArgs& a, int NW, int wave, int lane, const ProRegs& X,
                                                 uint32_t* L, const LdsPlan& P) {
  const int nb = a.nb, row = lane >> 4, j = lane & 15;
  if constexpr (PRO == PRO_Q8K) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      if (4 * NW * r + 4 * wave < nb) {  // uniform in the wave
        const int b = 4 * NW * r + 4 * wave + row;
        store_xblock(L, P, min(b, nb - 1), j, b < nb, X.q[r], X.d[r], X.bs[r]);
      }
    }
  } else {
    constexpr bool norm = (PRO == PRO_NORM_AWAY || PRO == PRO_NORM_EVEN);
    constexpr bool away = (PRO == PRO_QUANT_AWAY || PRO == PRO_NORM_AWAY);
    constexpr bool attn = (PRO == PRO_ATTN_EVEN || PRO == PRO_ATTN_ONE);
    if constexpr (PRO == PRO_ATTN_EVEN) attn_combine(a, X, reinterpret_cast<float*>(L + P.u));
    if constexpr (PRO == PRO_ATTN_ONE)
      attn_xcd_heads(a, X.kv, X.aq, reinterpret_cast<float*>(L + P.u), reinterpret_cast<float*>(L + P.at));
    float rms = 1.0f;
    if constexpr (norm) {
      // thread t's partial runs over x[t], x[t+256], ... (multiply then add)
      float p = 0.0f;
      if (wave < 4) {
#pragma unroll
        for (int jj = 0; jj < MAX_NB; ++jj)
          if (jj < nb) p = p + X.xp[jj] * X.xp[jj];
      }
      rms = block_rms_1sync(p, nb * QK_K, a.eps, reinterpret_cast<float*>(L + P.red));
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      if (4 * NW * r + 4 * wave < nb) {  // uniform in the wave: waves past the blocks skip
        const int b = 4 * NW * r + 4 * wave + row;
        float v[16];
        f32x4 xv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (attn)
            xv[i] = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(L + P.u) + min(b, nb - 1) * QK_K +
                                                    16 * j + 4 * i);
          else
            xv[i] = X.x[r][i];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[4 * i] = xv[i].x;
          v[4 * i + 1] = xv[i].y;
          v[4 * i + 2] = xv[i].z;
          v[4 * i + 3] = xv[i].w;
        }
        if constexpr (norm) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            v[4 * i] = (v[4 * i] * rms) * X.g[r][i].x;
            v[4 * i + 1] = (v[4 * i + 1] * rms) * X.g[r][i].y;
            v[4 * i + 2] = (v[4 * i + 2] * rms) * X.g[r][i].z;
            v[4 * i + 3] = (v[4 * i + 3] * rms) * X.g[r][i].w;
          }
        }
        u32x4 packed;
        float d;
        int gsum;
        quant_block_row16(v, away, packed, d, gsum);
        store_xblock(L, P, min(b, nb - 1), j, b < nb, packed, d, gsum);
      }
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------- weight rows ----
// Weight types a kernel instance handles: Q4_K only, Q6_K only, or both (per
// region, e.g. a Q6_K attn_v beside Q4_K q and k).  A single-type instance
// holds only its own block registers.
enum { WT_Q4 = 0, WT_Q6 = 1, WT_MIX = 2 };
struct Region {
  const uint8_t* p0;
  const uint8_t* p1;
  const uint8_t* p2;
  const uint8_t* p3;
  float* out;
  int rows;
  int row0;  // first item of the region (region mode)
  int type;
};

__device__ __forceinline__ Region region_of(const GemvRegion& g) {
  return Region{g.w.p0, g.w.p1, g.w.p2, g.w.p3, g.out, g.rows, g.row0, g.w.type};
}

// One slot of a work item: region, row, and the row's position in each plane
// (block 0, chunk 0).  Rows past the region's end point at its last row, so
// every load stays inside the tensor; `valid` masks their results.
struct RowRef {
  const uint8_t* p0;
  const uint8_t* p1;
  const uint8_t* p2;
  const uint8_t* p3;
  float* out;
  size_t rs;  // rows * 16: bytes between consecutive chunk planes
  int reg;
  int r;
  bool valid;
  bool q4;  // wave-uniform
};

template <int WT>
__device__ __forceinline__ RowRef row_of(const GemvArgs& a, const Region& A, const Region& B, const Region& C,
                                         int S, int item, int s) {
  RowRef t;
  int reg, r, rows;
  if (a.pair) {
    // slots 0..S/2-1 from region 0, the rest from region 1, same rows
    const int half = S / 2;
    reg = s < half ? 0 : 1;
    r = item * half + (s < half ? s : s - half);
    rows = a.total_rows;
    t.q4 = A.type == MCPM_TYPE_Q4_K;  // both regions share the type
  } else {
    reg = 0;
    if (a.nreg > 1 && item >= B.row0) reg = 1;
    if (a.nreg > 2 && item >= C.row0) reg = 2;
    r = (item - MCPM_PICK(reg, A, B, C, row0)) * S + s;
    rows = MCPM_PICK(reg, A, B, C, rows);
    t.q4 = MCPM_PICK(reg, A, B, C, type) == MCPM_TYPE_Q4_K;
  }
  if constexpr (WT != WT_MIX) t.q4 = (WT == WT_Q4);
  t.valid = r < rows && s < S;
  const size_t rr = static_cast<size_t>(min(r, rows - 1));
  t.reg = reg;
  t.r = r;
  t.rs = static_cast<size_t>(rows) * 16;
  t.p0 = MCPM_PICK(reg, A, B, C, p0) + rr * 16;
  t.p1 = MCPM_PICK(reg, A, B, C, p1) + rr * 16;
  t.p2 = MCPM_PICK(reg, A, B, C, p2) + rr * 16;
  t.p3 = MCPM_PICK(reg, A, B, C, p3) + rr * 2;
  t.out = MCPM_PICK(reg, A, B, C, out);
  return t;
}

// One block of one row in registers.  Q4_K: w[0..7] quant chunks, w[8]
// header.  Q6_K: w[0..7] ql chunks, w[8..11] qh chunks, w[12] scales, d.
template <int WT>
struct Blk {
  u32x4 w[WT == WT_Q4 ? 9 : 13];
  uint32_t d;
};

template <int WT>
__device__ __forceinline__ void load_blk(Blk<WT>& K, const RowRef& t, int b) {
  const size_t rs = t.rs;
  if constexpr (WT == WT_Q4) {
    const uint8_t* q = t.p0 + static_cast<size_t>(b) * 8 * rs;
#pragma unroll
    for (int c = 0; c < 8; ++c) K.w[c] = ld_stream4(q + c * rs);
    K.w[8] = ld_stream4(t.p1 + static_cast<size_t>(b) * rs);
    return;
  } else {
  if (WT == WT_MIX && t.q4) {
    const uint8_t* q = t.p0 + static_cast<size_t>(b) * 8 * rs;
#pragma unroll
    for (int c = 0; c < 8; ++c) K.w[c] = ld_stream4(q + c * rs);
    K.w[8] = ld_stream4(t.p1 + static_cast<size_t>(b) * rs);
  } else {
    const uint8_t* ql = t.p0 + static_cast<size_t>(b) * 8 * rs;
    const uint8_t* qh = t.p1 + static_cast<size_t>(b) * 4 * rs;
#pragma unroll
    for (int c = 0; c < 8; ++c) K.w[c] = ld_stream4(ql + c * rs);
#pragma unroll
    for (int c = 0; c < 4; ++c) K.w[8 + c] = ld_stream4(qh + c * rs);
    K.w[12] = ld_stream4(t.p2 + static_cast<size_t>(b) * rs);
    K.d = ld_stream_u16(t.p3 + static_cast<size_t>(b) * (rs / 8));
  }
  }
}

// dword i of the vectors starting at w (i a compile-time constant after unrolling)
__device__ __forceinline__ uint32_t dw(const u32x4* w, int i) {
  const u32x4 v = w[i >> 2];
  return (i & 3) == 0 ? v.x : (i & 3) == 1 ? v.y : (i & 3) == 2 ? v.z : v.w;
}

__device__ __forceinline__ int mad24(int a, int b, int c) { return __mul24(a, b) + c; }

// c + the four signed byte products of a and b (v_dot4c: the accumulator is
// the destination, so a running sum costs no extra instruction)
__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

// bytes k and k+1 of w as a pair of (zero-extended) 16-bit lanes
__device__ __forceinline__ uint32_t byte_pair(uint32_t w, int k) {
  return __builtin_amdgcn_perm(0u, w, 0x0c000c00u | (static_cast<uint32_t>(k + 1) << 16) | static_cast<uint32_t>(k));
}

__device__ __forceinline__ int dot2(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot2(__builtin_bit_cast(i16x2, a), __builtin_bit_cast(i16x2, b), c, false);
}

// Eight lane sums of a Q4_K block against Q8_K block xs (64 dwords), and the
// block's min sum over the 8 sub-blocks of mn_g*(bsums[2g]+bsums[2g+1]) (xbp:
// those pair sums as i16 pairs).  Native quant dword 8j+m holds, per byte,
// sub-block 2j (low nibble) and 2j+1 (high nibble) at positions 4m..4m+3.
//
// isum[m] = sum_k sc_k*D_k over sub-blocks k (D_k: lane m's 4-byte dot) is
// formed by summation by parts: with running dots P_k = D_0 + .. + D_k,
// isum[m] = sum_{k<7} (sc_k - sc_{k+1})*P_k + sc_7*P_7, the same integer.  The
// running dot is the dot instruction's own accumulator.
template <int WT>
__device__ __forceinline__ void q4k_rowblock(const Blk<WT>& K, const uint32_t* __restrict__ xs,
                                             const uint32_t* __restrict__ xbp, int (&is)[8], int& ms) {
  const uint32_t s0 = K.w[8].y, s1 = K.w[8].z, s2 = K.w[8].w;
  // scales (sc) and mins (mn) of sub-blocks 0..3 and 4..7, one per byte
  const uint32_t sc_lo = s0 & 0x3f3f3f3fu;
  const uint32_t sc_hi = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
  const uint32_t mn_lo = s1 & 0x3f3f3f3fu;
  const uint32_t mn_hi = ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u);
  int sc[8], cf[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    sc[k] = static_cast<int>(__builtin_amdgcn_ubfe(sc_lo, 8 * k, 8));
    sc[4 + k] = static_cast<int>(__builtin_amdgcn_ubfe(sc_hi, 8 * k, 8));
  }
#pragma unroll
  for (int k = 0; k < 7; ++k) cf[k] = sc[k] - sc[k + 1];
  cf[7] = sc[7];
  int P[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const u32x4 xe0 = *reinterpret_cast<const u32x4*>(xs + 16 * j);
    const u32x4 xe1 = *reinterpret_cast<const u32x4*>(xs + 16 * j + 4);
    const u32x4 xo0 = *reinterpret_cast<const u32x4*>(xs + 16 * j + 8);
    const u32x4 xo1 = *reinterpret_cast<const u32x4*>(xs + 16 * j + 12);
    const uint32_t xe[8] = {xe0.x, xe0.y, xe0.z, xe0.w, xe1.x, xe1.y, xe1.z, xe1.w};
    const uint32_t xo[8] = {xo0.x, xo0.y, xo0.z, xo0.w, xo1.x, xo1.y, xo1.z, xo1.w};
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const uint32_t q = dw(K.w, 8 * j + m);
      P[m] = dot4(q & 0x0f0f0f0fu, xe[m], j == 0 ? 0 : P[m]);
      is[m] = j == 0 ? __mul24(cf[0], P[m]) : mad24(cf[2 * j], P[m], is[m]);
      P[m] = dot4((q >> 4) & 0x0f0f0f0fu, xo[m], P[m]);
      is[m] = mad24(cf[2 * j + 1], P[m], is[m]);
    }
  }
  const u32x4 bp = *reinterpret_cast<const u32x4*>(xbp);
  int v = dot2(byte_pair(mn_lo, 0), bp.x, 0);
  v = dot2(byte_pair(mn_lo, 2), bp.y, v);
  v = dot2(byte_pair(mn_hi, 0), bp.z, v);
  ms = dot2(byte_pair(mn_hi, 2), bp.w, v);
}

// Eight lane sums of a Q6_K block (codes kept in [0, 63], the -32 applied as
// 32*(bsums[2m]*sc[2m] + bsums[2m+1]*sc[2m+1])).  For half h and lane m:
// ql dwords 16h+m, 16h+8+m, qh dword 8h+m, activations 32h+8g+m (g = 0..3),
// scale 8h+2g+(m>=4).  Lane m's eight terms (h, g) in that order are summed
// by parts over running dots as in q4k_rowblock, with the scale sequence of
// its half of the lanes (m < 4 or m >= 4).
template <int WT>
__device__ __forceinline__ void q6k_rowblock(const Blk<WT>& K, const uint32_t* __restrict__ xs,
                                             const uint32_t* __restrict__ xbs, int (&is)[8]) {
  int sc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) sc[i] = __builtin_amdgcn_sbfe(static_cast<int>(dw(&K.w[12], i >> 2)), 8 * (i & 3), 8);
  // cf[hi][k]: term k = 4h+g has scale sc[8h+2g+hi]
  int cf[2][8];
#pragma unroll
  for (int hi = 0; hi < 2; ++hi) {
#pragma unroll
    for (int k = 0; k < 7; ++k) cf[hi][k] = sc[8 * (k >> 2) + 2 * (k & 3) + hi] - sc[8 * ((k + 1) >> 2) + 2 * ((k + 1) & 3) + hi];
    cf[hi][7] = sc[8 + 6 + hi];
  }
  int P[8];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t xv[4][8];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const u32x4 x0 = *reinterpret_cast<const u32x4*>(xs + 32 * h + 8 * g);
      const u32x4 x1 = *reinterpret_cast<const u32x4*>(xs + 32 * h + 8 * g + 4);
      xv[g][0] = x0.x;
      xv[g][1] = x0.y;
      xv[g][2] = x0.z;
      xv[g][3] = x0.w;
      xv[g][4] = x1.x;
      xv[g][5] = x1.y;
      xv[g][6] = x1.z;
      xv[g][7] = x1.w;
    }
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int hi = (m >= 4) ? 1 : 0;
      const uint32_t a0 = dw(K.w, 16 * h + m), a1 = dw(K.w, 16 * h + 8 + m), hb = dw(&K.w[8], 8 * h + m);
      const uint32_t q0 = (a0 & 0x0f0f0f0fu) | ((hb << 4) & 0x30303030u);
      const uint32_t q1 = (a1 & 0x0f0f0f0fu) | ((hb << 2) & 0x30303030u);
      const uint32_t q2 = ((a0 >> 4) & 0x0f0f0f0fu) | (hb & 0x30303030u);
      const uint32_t q3 = ((a1 >> 4) & 0x0f0f0f0fu) | ((hb >> 2) & 0x30303030u);
      P[m] = dot4(q0, xv[0][m], h == 0 ? 0 : P[m]);
      int v = h == 0 ? __mul24(cf[hi][0], P[m]) : mad24(cf[hi][4], P[m], is[m]);
      P[m] = dot4(q1, xv[1][m], P[m]);
      v = mad24(cf[hi][4 * h + 1], P[m], v);
      P[m] = dot4(q2, xv[2][m], P[m]);
      v = mad24(cf[hi][4 * h + 2], P[m], v);
      P[m] = dot4(q3, xv[3][m], P[m]);
      is[m] = mad24(cf[hi][4 * h + 3], P[m], v);
    }
  }
  int bsv[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4 t = *reinterpret_cast<const u32x4*>(xbs + 4 * i);
    bsv[4 * i] = static_cast<int>(t.x);
    bsv[4 * i + 1] = static_cast<int>(t.y);
    bsv[4 * i + 2] = static_cast<int>(t.z);
    bsv[4 * i + 3] = static_cast<int>(t.w);
  }
#pragma unroll
  for (int m = 0; m < 8; ++m) is[m] -= 32 * mad24(bsv[2 * m], sc[2 * m], __mul24(bsv[2 * m + 1], sc[2 * m + 1]));
}

__device__ __forceinline__ float hsum8(const float (&acc)[8]) {
  return ((acc[0] + acc[4]) + (acc[2] + acc[6])) + ((acc[1] + acc[5]) + (acc[3] + acc[7]));
}

// Work groups are dispatched round-robin over the 8 XCDs (work group b on
// XCD b % 8), each with its own L2.  A GRP item's rows are 16-byte runs of
// every chunk plane that do not fill whole 128-byte lines, so a line is
// shared with the neighbouring item: giving each XCD a contiguous range of
// items (this bijection of [0, G)) lets the neighbour's half come from the
// same L2 instead of HBM.
__device__ __forceinline__ int xcd_contiguous(int b, int G) {
  const int x = b & 7, k = b >> 3;
  const int q = G >> 3, r = G & 7;  // XCD x runs q + (x < r) work groups
  return x * q + min(x, r) + k;
}

// ---------------------------------------------------------------- kernel ---
// TILE: S slots per item, KB steps per item, 4 waves.  ROW: S = 64, KB = nb,
// 4..8 waves.  TILE's bound of 4 waves lets a wave hold up to 512 registers
// (VGPRs and AGPRs), so its step registers never go to scratch.
// GRP (with TILE): the item belongs to the work group, its pairs spread over
// the 4 waves (pair q = lane + 64*wave + 256*k), one chain area in LDS that
// wave 0 runs after a work-group barrier.  It gives each SIMD one step where
// a wave-sized item would need two (the down projection: 23 blocks).
// The (item, step) sequence of one wave of a launch, with the launch's work
// group index and count given (a kernel's own, or a fused kernel's virtual
// ones), and the epilogue inputs its rows need.
template <int EPI, bool TILE, int WT, bool GRP, int COH>
struct GemvPlan {
  const GemvArgs& a;
  int n_items, S, KB, lane, wave, NW, nb, stride, first, n_steps, pos;
  float invS;
  Region A, B, C;

  __device__ __forceinline__ GemvPlan(const GemvArgs& a_, int n_items_, int S_, int KB_, int vb, int vg)
      : a(a_), n_items(n_items_), S(S_), KB(KB_) {
    lane = threadIdx.x & 63;
    wave = sgpr(static_cast<int>(threadIdx.x >> 6));
    NW = TILE ? GEMV_TILE_WAVES : static_cast<int>(blockDim.x >> 6);
    nb = a.nb;
    stride = GRP ? vg : vg * NW;
    A = region_of(a.reg[0]);
    B = region_of(a.reg[1]);
    C = region_of(a.reg[2]);
    // This wave's steps: item first + (t / KB) * stride, step t % KB.  Steps
    // past the last re-read the last one (cached, results unused), so every
    // load is issued unconditionally and no wait depends on a branch.
    first = GRP ? xcd_contiguous(vb, vg) : vb * NW + wave;
    const int n_mine = first < n_items ? (n_items - 1 - first) / stride + 1 : 0;
    n_steps = n_mine * KB;
    invS = 1.0f / static_cast<float>(S);
    pos = (EPI == EPI_QKV) ? a.state[1] : 0;
  }

  // slot and block of this lane at step k of an item
  __device__ __forceinline__ void slot_at(int k, int& s, int& b) const {
    if constexpr (TILE) {
      const int q = GRP ? lane + 64 * wave + 256 * k : lane + 64 * k;
      const int bq = static_cast<int>((static_cast<float>(q) + 0.5f) * invS);  // q / S, exact for q < 2^16
      s = q - bq * S;
      b = bq;
    } else {
      s = lane;
      b = k;
    }
  }
  __device__ __forceinline__ RowRef ref_at(int t, int& b, int& s) const {
    const int tt = min(t, max(n_steps - 1, 0));
    const int it = n_steps > 0 ? first + (tt / KB) * stride : 0;
    slot_at(tt % KB, s, b);
    return row_of<WT>(a, A, B, C, S, it, s);
  }
  // Epilogue inputs of the row this lane finishes (ROW: its row; TILE: slot
  // `lane`), loaded with each step's weights so the epilogue reads no memory:
  // the residual (RESID) or the RoPE cos/sin (QKV).  Every step loads them,
  // at clamped indices, so no load depends on a branch.
  __device__ __forceinline__ void prefetch_epi(int t, float2& e) const {
    const int tt = min(t, max(n_steps - 1, 0));
    const int it = n_steps > 0 ? first + (tt / KB) * stride : 0;
    const RowRef te = row_of<WT>(a, A, B, C, S, it, min(lane, S - 1));
    if constexpr (EPI == EPI_RESID) {
      e.x = a.resid[min(te.r, a.total_rows - 1)];
    } else if constexpr (EPI == EPI_QKV) {
      const int i = te.r % a.head_dim;
      e = a.rope_cs[static_cast<size_t>(pos) * (a.head_dim / 2) + (i >> 1)];
    }
  }
};

// A wave's first step (weights and epilogue inputs), loaded ahead: a fused
// kernel issues it before waiting for the producer of the activations.
template <int WT>
struct FirstStep {
  Blk<WT> K;
  float2 e;
  RowRef t;
  int b, s;
};

template <int EPI, bool TILE, int WT, bool GRP, int COH>
__device__ __forceinline__ void gemv_first_step(const GemvPlan<EPI, TILE, WT, GRP, COH>& pl, FirstStep<WT>& f) {
  f.e = make_float2(0.0f, 0.0f);
  f.t = pl.ref_at(0, f.b, f.s);
  load_blk(f.K, f.t, min(f.b, pl.nb - 1));
  pl.prefetch_epi(0, f.e);
}

// One GEMV launch's work for virtual work group vb of vg: the body of k_gemv,
// and a phase of the fused kernels.  COH: the activations come from other
// work groups of the same launch and the outputs go to them (sc1 loads and
// stores); PRE: the first step was loaded by gemv_first_step (in `pre`).
// Ends with the wave's last stores issued (not waited for).
template <int PRO, int EPI, bool TILE, int WT, bool GRP = false, int COH = 0, bool PRE = false>
__device__ __forceinline__ void gemv_core(const GemvArgs& a, int n_items, int S, int KB, int vb, int vg, uint32_t* L,
                                          const FirstStep<WT>* pre) {
  static_assert(TILE || !GRP, "GRP is a TILE shape");
  const GemvPlan<EPI, TILE, WT, GRP, COH> pl(a, n_items, S, KB, vb, vg);
  const int lane = pl.lane, wave = pl.wave, NW = pl.NW, nb = pl.nb;
  const LdsPlan P = lds_plan(nb, S, TILE, lds_attn<PRO>(), GRP ? 1 : NW);
  const int stride = pl.stride, first = pl.first, n_steps = pl.n_steps, pos = pl.pos;
  const Region &A = pl.A, &B = pl.B, &C = pl.C;
  auto ref_at = [&](int t, int& b, int& s) { return pl.ref_at(t, b, s); };
  auto prefetch_epi = [&](int t, float2& e) { pl.prefetch_epi(t, e); };

  ProRegs X;
  prologue_load<PRO, COH>(a, NW, wave, lane, X);
  // A CU's vector loads return in issue order, so an activation load queued
  // behind weight loads (HBM) waits for them.  Every wave's activation loads
  // go first: a bare barrier (no wait for the data) before any weight load.
  __builtin_amdgcn_s_barrier();
  Blk<WT> K0, K1;
  float2 e0 = make_float2(0.0f, 0.0f), e1 = make_float2(0.0f, 0.0f);
  int b0, s0, b1, s1;
  RowRef t0, t1;
  if constexpr (PRE) {
    K0 = pre->K;
    e0 = pre->e;
    t0 = pre->t;
    b0 = pre->b;
    s0 = pre->s;
  } else {
    t0 = ref_at(0, b0, s0);
    load_blk(K0, t0, min(b0, nb - 1));  // in flight during the prologue
    prefetch_epi(0, e0);
  }
  prologue_compute<PRO>(a, NW, wave, lane, X, L, P);

  float acc[8], accm = 0.0f;
#pragma unroll
  for (int m = 0; m < 8; ++m) acc[m] = 0.0f;
  float best_v = -__builtin_inff();
  int best_i = 0x7fffffff;
  uint32_t* chain = L + P.u + (GRP ? 0 : wave * (nb * S * 12));  // TILE: entry (b, s) at (b*S + s)*12

  // the epilogue for row value v of slot s of item `it`; lanes with s >= S
  // or an invalid row only take part in the shuffles before it
  auto epilogue = [&](int it, int s, float v, float partner, float up, float2 e) {
    const RowRef t = row_of<WT>(a, A, B, C, S, it, min(s, S - 1));
    const bool writer = s < S && t.valid;
    const int r = t.r;
    auto put = [](float* p, float x) {
      if constexpr ((COH & COH_OUT) != 0) st_coh(p, x);
      else *p = x;
    };
    if constexpr (EPI == EPI_STORE) {
      if (writer) put(t.out + r, v);
    } else if constexpr (EPI == EPI_RESID) {
      if (writer) put(a.resid + r, e.x + v);
    } else if constexpr (EPI == EPI_SWIGLU) {
      if (writer && s < S / 2) {
        const float silu = v / (1.0f + exp_f32(-v));
        put(a.h_out + r, silu * up);
      }
    } else if constexpr (EPI == EPI_QKV) {
      // adjacent-pair RoPE (src/ops/ops.cpp:502-516) on q (region 0) and k
      // (region 1); k and v rows go to the KV cache at pos.
      if (writer) {
        if (t.reg < 2) {
          const int i = r % a.head_dim;
          const float2 cs = e;
          float o;
          if ((i & 1) == 0) o = v * cs.x - partner * cs.y;
          else o = partner * cs.y + v * cs.x;
          if (t.reg == 0) put(t.out + r, o);
          else put(a.k_cache + static_cast<size_t>(pos) * a.kvd + r, o);
        } else {
          put(a.v_cache + static_cast<size_t>(pos) * a.kvd + r, v);
        }
      }
    } else if constexpr (EPI == EPI_LOGITS) {
      if (writer) {
        put(t.out + r, v);
        if (v > best_v || (v == best_v && r < best_i)) {
          best_v = v;
          best_i = r;
        }
      }
    }
  };

  // integer work of one step, then the float chain (ROW) or its LDS entry
  // (TILE); the item's last step finishes its rows
  auto consume = [&](const Blk<WT>& Kb, float2 e, const RowRef& t, int t_idx, int b, int s) {
    const int k = t_idx % KB;
    const int it = first + (t_idx / KB) * stride;
    const int bc = min(b, nb - 1);
    int is[8], ms = 0;
    float ds, dm = 0.0f;
    const float xdv = __uint_as_float(L[P.xd + bc]);
    if (WT == WT_Q4 || (WT == WT_MIX && t.q4)) {
      q4k_rowblock(Kb, L + P.xs + bc * 68, L + P.xbp + bc * 4, is, ms);
      ds = xdv * fp16_to_fp32(static_cast<uint16_t>(Kb.w[8].x & 0xffffu));
      dm = xdv * fp16_to_fp32(static_cast<uint16_t>(Kb.w[8].x >> 16));
    } else {
      if constexpr (WT != WT_Q4) {
        q6k_rowblock(Kb, L + P.xs + bc * 68, L + P.xbs + bc * 16, is);
        ds = xdv * fp16_to_fp32(static_cast<uint16_t>(Kb.d & 0xffffu));
      }
    }
    if constexpr (!TILE) {
      if (k == 0) {
#pragma unroll
        for (int m = 0; m < 8; ++m) acc[m] = 0.0f;
        accm = 0.0f;
      }
#pragma unroll
      for (int m = 0; m < 8; ++m) acc[m] = __builtin_fmaf(ds, static_cast<float>(is[m]), acc[m]);
      accm = __builtin_fmaf(-dm, static_cast<float>(ms), accm);
      if (k == KB - 1) {
        float v = hsum8(acc);
        if (t.q4) v = v + accm;
        const float partner = __shfl(v, lane ^ 1);
        const float up = __shfl(v, (lane + 32) & 63);
        epilogue(it, lane, v, partner, up, e);
      }
    } else {
      if (b < nb) {
        u32x4* e = reinterpret_cast<u32x4*>(chain + (b * S + s) * 12);
        e[0] = u32x4{static_cast<uint32_t>(is[0]), static_cast<uint32_t>(is[1]), static_cast<uint32_t>(is[2]),
                     static_cast<uint32_t>(is[3])};
        e[1] = u32x4{static_cast<uint32_t>(is[4]), static_cast<uint32_t>(is[5]), static_cast<uint32_t>(is[6]),
                     static_cast<uint32_t>(is[7])};
        e[2] = u32x4{__float_as_uint(ds), __float_as_uint(dm), static_cast<uint32_t>(ms), 0u};
      }
      if (k == KB - 1) {
        // GRP: every wave's entries are in before wave 0 runs the chain
        if constexpr (GRP) __syncthreads();
        else wave_sync();
        if (!GRP || wave == 0) {
          // 4 lanes per row (lane = 4*row + c, S/16 passes) run the chain, lane c
          // the accumulators of lane sums c and c+4; the row values go to vrow
          // for the epilogue's RoPE and gate/up partners
          const int c = lane & 3;
          float* vrow = reinterpret_cast<float*>(L + P.vrow) + wave * 64;
#pragma unroll 1
          for (int pass = 0; pass * 16 < S; ++pass) {
            const int sr = pass * 16 + (lane >> 2);
            const int src = min(sr, S - 1);
            float a0 = 0.0f, a1 = 0.0f, am = 0.0f;
            // CHAIN_BATCH blocks' entries read at once (one LDS round trip for
            // up to 12 blocks), then their fma steps in order
#pragma unroll 1
            for (int bq = 0; bq < nb; bq += CHAIN_BATCH) {
              int i0[CHAIN_BATCH], i1[CHAIN_BATCH];
              f32x4 dv[CHAIN_BATCH];  // (d_x*d_w, d_x*dmin_w, minsum, -)
#pragma unroll
              for (int k = 0; k < CHAIN_BATCH; ++k) {
                const uint32_t* e = chain + (min(bq + k, nb - 1) * S + src) * 12;
                i0[k] = static_cast<int>(e[c]);
                i1[k] = static_cast<int>(e[c + 4]);
                dv[k] = *reinterpret_cast<const f32x4*>(e + 8);
              }
#pragma unroll
              for (int k = 0; k < CHAIN_BATCH; ++k) {
                if (bq + k < nb) {
                  a0 = __builtin_fmaf(dv[k].x, static_cast<float>(i0[k]), a0);
                  a1 = __builtin_fmaf(dv[k].x, static_cast<float>(i1[k]), a1);
                  am = __builtin_fmaf(-dv[k].y, static_cast<float>(__float_as_int(dv[k].z)), am);
                }
              }
            }
            // ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) on lane c == 0, the partner
            // lanes 4r+2 and 4r+1 read by DPP row shifts
            float v = a0 + a1;
            v = v + dpp_f<0x102>(v);  // row_shl:2
            v = v + dpp_f<0x101>(v);  // row_shl:1
            if (t.q4) v = v + am;
            if (c == 0 && sr < S) vrow[sr] = v;
          }
          wave_sync();
          const int se = min(lane, S - 1);
          const float v = vrow[se];
          const float partner = vrow[(se ^ 1) < S ? (se ^ 1) : se];
          const float up = vrow[(se + S / 2) % S];
          wave_sync();  // every read of the chain area precedes the next item's entries
          epilogue(it, lane, v, partner, up, e);
        }
        if constexpr (GRP) __syncthreads();  // wave 0's chain reads precede the next item's entries
      }
    }
  };

  // TILE waves of one or two steps (every launch whose items fit the grid)
  // take straight-line paths that load nothing past their last step: issuing
  // a block's 9-13 vector loads holds a wave for ~0.6-1 us, so a re-read of
  // a clamped step is not free.  (Loads under a branch inside the loop would
  // make the compiler's wait at the join cover the loads of both paths.)
  if (TILE && n_steps == 1) {
    consume(K0, e0, t0, 0, b0, s0);
  } else if (TILE && n_steps == 2) {
    t1 = ref_at(1, b1, s1);
    prefetch_epi(1, e1);
    load_blk(K1, t1, min(b1, nb - 1));
    consume(K0, e0, t0, 0, b0, s0);
    consume(K1, e1, t1, 1, b1, s1);
  } else {
    // two register sets used in turn: a copy between them would wait for the
    // loads still landing in the source
    for (int t = 0; t < n_steps; t += 2) {
      t1 = ref_at(t + 1, b1, s1);
      prefetch_epi(t + 1, e1);
      load_blk(K1, t1, min(b1, nb - 1));
      consume(K0, e0, t0, t, b0, s0);
      if (t + 1 >= n_steps) break;
      t0 = ref_at(t + 2, b0, s0);
      prefetch_epi(t + 2, e0);
      load_blk(K0, t0, min(b0, nb - 1));
      consume(K1, e1, t1, t + 1, b1, s1);
    }
  }

  if constexpr (EPI == EPI_LOGITS) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(best_v, o);
      const int oi = __shfl_xor(best_i, o);
      if (ov > best_v || (ov == best_v && oi < best_i)) {
        best_v = ov;
        best_i = oi;
      }
    }
    if (lane == 0) a.argmax_part[vb * NW + wave] = make_float2(best_v, __int_as_float(best_i));
  }
}

template <int PRO, int EPI, bool TILE, int WT, bool GRP = false>
__global__ void __launch_bounds__(64 * (TILE ? GEMV_TILE_WAVES : GEMV_MAX_WAVES))
    k_gemv(const GemvArgs a, int n_items, int S, int KB) {
  extern __shared__ uint32_t L[];
  gemv_core<PRO, EPI, TILE, WT, GRP>(a, n_items, S, KB, static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x),
                                     L, nullptr);
}

// --------------------------------------------------------- fused kernels ----
// A grid barrier inside one launch whose work groups are all resident (grid
// <= CUs, one work group per CU): eight arrival counters, one per XCD (work
// group b runs on XCD b % 8 and arrives on counter b % 8), 256 bytes apart,
// and a launch count `gen` that work group 0 advances after the launch's
// last barrier (every work group has read it by then).  Barrier k of launch
// gen waits until counter x reaches (gen*nbar + k + 1) * (work groups on XCD
// x), compared by signed difference so that the counters may wrap.  Every
// wait is bounded: past the spin limit, or when another work group has given
// up, it sets the error word and returns false, and the kernel returns.
__device__ __forceinline__ unsigned ld_coh_u(const unsigned* p) {
  return __hip_atomic_load(const_cast<unsigned*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Arrival: every wave's outputs acknowledged (all its memory operations
// complete: issue no loads meant to overlap the wait before this), then one
// arrival per work group.
__device__ __forceinline__ void grid_arrive(const GridSync& g) {
  wait_stores();
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(g.ctr + 64 * (blockIdx.x & 7), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits for every work group's arrival at barrier k of launch gen; loads
// issued between grid_arrive and this call overlap the wait.
__device__ bool grid_wait(const GridSync& g, unsigned gen, int nbar, int k) {
  __shared__ int s_ok;
  const int G = static_cast<int>(gridDim.x);
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const unsigned round = gen * static_cast<unsigned>(nbar) + static_cast<unsigned>(k) + 1u;
    const unsigned members = static_cast<unsigned>(G / 8 + (lane < G % 8 ? 1 : 0));
    bool ok = true;
    unsigned spins = 0;
    for (;;) {
      bool mine = true;
      if (lane < 8) mine = static_cast<int>(ld_coh_u(g.ctr + 64 * lane) - round * members) >= 0;
      if (__all(mine)) break;
      if (++spins > g.spin_limit || ld_coh_u(g.err)) {
        if (lane == 0) __hip_atomic_store(g.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = false;
        break;
      }
    }
    if (lane == 0) s_ok = ok;
  }
  __syncthreads();
  return s_ok;
}

// The FFN block of one layer in one launch (src/model.cpp:195-225): gate/up
// (RMSNorm + Q8_K prologue, SwiGLU epilogue, h written through), then the
// down projection (Q8_K of h, residual add).  Each work group loads its first
// down step (weights and residual) before the grid barrier, so that latency
// overlaps the barrier instead of following it.  Both phases are TILE shapes
// of 4 waves; virtual work group counts gu_grid and dn_grid <= the grid.
template <int WT_DN, bool GRP_DN>
__global__ void __launch_bounds__(64 * GEMV_TILE_WAVES)
    k_ffn_fused(const GemvArgs gu, int gu_items, int gu_S, int gu_KB, int gu_grid, const GemvArgs dn, int dn_items,
                int dn_S, int dn_KB, int dn_grid, GridSync gs) {
  extern __shared__ uint32_t L[];
  const int b = static_cast<int>(blockIdx.x);
  __shared__ unsigned s_gen;
  if (threadIdx.x == 0) s_gen = ld_coh_u(gs.gen);
  // gate/up: x from the previous launch; h written through for the others
  if (b < gu_grid)
    gemv_core<PRO_NORM_AWAY, EPI_SWIGLU, true, WT_Q4, false, COH_OUT>(gu, gu_items, gu_S, gu_KB, b, gu_grid, L,
                                                                      nullptr);
  grid_arrive(gs);  // also makes s_gen visible to every wave
  const unsigned gen = s_gen;
  // the first down step's weights and residual, in flight during the wait
  // (issued earlier, at the start, they slow gate/up down more than they save)
  const GemvPlan<EPI_RESID, true, WT_DN, GRP_DN, COH_IN> pl(dn, dn_items, dn_S, dn_KB, b, dn_grid);
  FirstStep<WT_DN> pre;
  if (b < dn_grid) gemv_first_step(pl, pre);
  if (!grid_wait(gs, gen, 1, 0)) return;
  if (b == 0 && threadIdx.x == 0) __hip_atomic_fetch_add(gs.gen, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // down: h from the other work groups; each row's residual read and written by one lane
  if (b < dn_grid)
    gemv_core<PRO_QUANT_AWAY, EPI_RESID, true, WT_DN, GRP_DN, COH_IN, true>(dn, dn_items, dn_S, dn_KB, b, dn_grid,
                                                                            L, &pre);
}

// QKV and attention of one layer in one launch (src/model.cpp:178-195): the
// QKV GEMV (RMSNorm + Q8_K prologue, RoPE; q and the K and V rows at pos
// written through for the other work groups), a grid barrier, then
// k_attention's splits, work group b taking splits b, b + G, ... (split it:
// kv head it % n_kv_heads, split it / n_kv_heads).  A work group issues its
// first split's K and V loads before the barrier, so their latency overlaps
// the wait, all but the row at pos, which this launch writes: that row is
// read only after the barrier.  Work groups without a split leave after
// arriving (work group 0 waits, then advances the barrier's launch count).
template <int WT, int HDM>
__global__ void __launch_bounds__(64 * GEMV_TILE_WAVES)
    k_qkv_attn(const GemvArgs qa, int q_items, int q_S, int q_KB, int q_grid, const AttnArgs at, GridSync gs) {
  extern __shared__ __attribute__((aligned(16))) uint32_t LQA[];
  const int b = static_cast<int>(blockIdx.x), G = static_cast<int>(gridDim.x);
  __shared__ unsigned s_gen;
  if (threadIdx.x == 0) s_gen = ld_coh_u(gs.gen);
  if (b < q_grid)
    gemv_core<PRO_NORM_AWAY, EPI_QKV, true, WT, false, COH_OUT>(qa, q_items, q_S, q_KB, b, q_grid, LQA, nullptr);
  grid_arrive(gs);  // also makes s_gen visible to every wave
  const unsigned gen = s_gen;
  const int T = at.state[1] + 1;
  const int nch = (T + ATTN_CHUNK - 1) / ATTN_CHUNK;
  const int n_items = at.n_kv_heads * attn_splits(nch);
  if (b >= n_items && b != 0) return;
  AttnRegs<HDM / 16> R;
  if (b < n_items) {
    const int r4 = at.head_dim / 4;
    attn_load_chunk<HDM / 16, true>(R, at.kc, at.vc, (b / at.n_kv_heads) * attn_chunks_per_split(nch), T,
                              at.n_kv_heads * at.head_dim, static_cast<size_t>(b % at.n_kv_heads) * at.head_dim, r4,
                              ATTN_CHUNK * r4);
  }
  if (!grid_wait(gs, gen, 1, 0)) return;
  if (b == 0 && threadIdx.x == 0) __hip_atomic_fetch_add(gs.gen, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const AttnLds<HDM> S(reinterpret_cast<float*>(LQA));
  for (int it = b; it < n_items; it += G)
    attn_split<HDM, true>(at.q, at.kc, at.vc, T, it % at.n_kv_heads, it / at.n_kv_heads, at.n_heads, at.n_kv_heads,
                          at.head_dim, at.max_chunks, at.part_o, at.part_mz, S, R, it == b);
}

// ------------------------------------------------------------- dispatch ----

namespace {

struct Shape {
  bool tile;
  int S, KB;
  int NW;            // waves per work group
  bool grp = false;  // TILE items of a whole work group
};

int items_for(const GemvArgs& a, int S) {
  if (a.pair) return (a.total_rows + S / 2 - 1) / (S / 2);
  int n = 0;
  for (int i = 0; i < a.nreg; ++i) n += (a.reg[i].rows + S - 1) / S;
  return n;
}

// ROW: one work group per CU holding ceil(items / n_cu) waves (4..8), so
// every CU gets the same load (a second work group on some CUs only would run
// mostly after the first there, the oldest waves issuing first).
int waves_for(int items, int n_cu) { return std::min(GEMV_MAX_WAVES, std::max(4, (items + n_cu - 1) / n_cu)); }

// ROW when its 64-row items give every SIMD a wave.  Otherwise TILE with one
// wave per SIMD (4 per work group, at most one work group per CU): a second
// wave on a SIMD only adds its instructions to the first's, since a step's
// time is its integer work.  The fewest steps per item (KB) whose items fit
// 4*n_cu waves, then S a multiple of 4 (a step's rows of one block are 64-byte
// runs of each chunk plane), then the smallest S (least work per wave).  S is
// even where rows pair up (RoPE, gate/up) and S*nb <= 64*KB.
//
// GRP when those TILE items need two or more steps but work-group items (S
// rows, S*nb <= 256 pairs, one step per wave) fit one work group per CU; for
// launches whose epilogue needs no row pairs (residual, store).
//
// MCPM_GEMV_SHAPE_<QKV|OPROJ|GATE_UP|DOWN|LM|OTHER>="KB,S,NW" (KB 0: ROW; KB
// < 0: GRP with -KB steps; NW counts for ROW only, TILE always runs 4 waves)
// overrides the choice for one class of launch: a tuning aid for measuring
// shapes against each other.
const char* shape_env(int prologue, int epilogue) {
  const char* name = "MCPM_GEMV_SHAPE_OTHER";
  if (epilogue == EPI_QKV) name = "MCPM_GEMV_SHAPE_QKV";
  else if (epilogue == EPI_SWIGLU) name = "MCPM_GEMV_SHAPE_GATE_UP";
  else if (epilogue == EPI_LOGITS) name = "MCPM_GEMV_SHAPE_LM";
  else if (epilogue == EPI_RESID) name = prologue == PRO_QUANT_AWAY ? "MCPM_GEMV_SHAPE_DOWN" : "MCPM_GEMV_SHAPE_OPROJ";
  return std::getenv(name);
}

Shape pick_shape(const GemvArgs& a, int prologue, int epilogue, int n_cu) {
  const int nb = a.nb;
  const bool paired = a.pair || epilogue == EPI_QKV;
  const bool grp_ok = !paired && (epilogue == EPI_RESID || epilogue == EPI_STORE);
  if (const char* env = shape_env(prologue, epilogue)) {
    int kb = -1, s = 0, nw = 4;
    if (std::sscanf(env, "%d,%d,%d", &kb, &s, &nw) >= 1 && nw >= 4 && nw <= GEMV_MAX_WAVES) {
      if (kb == 0) return Shape{false, 64, nb, nw};
      if (kb > 0 && kb <= 4 && s >= 1 && s <= 64 && !(paired && s % 2) && s * nb <= 64 * kb)
        return Shape{true, s, kb, GEMV_TILE_WAVES};
      if (kb < 0 && kb >= -4 && grp_ok && s >= 1 && s <= 64 && s * nb <= 256 * -kb)
        return Shape{true, s, -kb, GEMV_TILE_WAVES, true};
    }
  }
  // the O projection (a residual epilogue after a ties-even or given Q8_K
  // input): work-group items of 16 rows (2.4B shape, 256-token decode: 9.4
  // -> 8.9 us per launch at contexts past 192, 696 -> 704 tok/s; 8, 12, 14,
  // 20, 24 and 32 rows and the one-wave items of 3-8 rows were slower)
  if (epilogue == EPI_RESID && prologue != PRO_QUANT_AWAY && grp_ok && 16 * nb <= 256 && items_for(a, 16) <= n_cu)
    return Shape{true, 16, 1, GEMV_TILE_WAVES, true};
  const int cap = 4 * n_cu;
  const int row_items = items_for(a, 64);
  if (row_items >= cap) return Shape{false, 64, nb, waves_for(row_items, n_cu)};
  for (int kb = 1; kb <= 4; ++kb) {
    Shape best{true, 0, kb, GEMV_TILE_WAVES};
    for (int S = paired ? 2 : 1; S * nb <= 64 * kb && S <= 64; S += paired ? 2 : 1) {
      if (items_for(a, S) > cap) continue;
      if (best.S == 0 || (S % 4 == 0 && best.S % 4 != 0)) best.S = S;
    }
    if (best.S) {
      // work-group items: the fewest rows per item that still give at most
      // one item per CU (the down projection of the 2.4B shape: 9 rows, 256
      // items, 8.7 -> 8.25 us per launch against the most rows one step
      // holds, 11; decode 702.9 -> 711.5 tok/s)
      int sg = std::min(64, 256 / nb);
      while (grp_ok && sg > 1 && items_for(a, sg - 1) <= n_cu) --sg;  // grp_ok: not paired (no S/2)
      if (kb >= 2 && grp_ok && sg >= 1 && items_for(a, sg) <= n_cu) return Shape{true, sg, 1, GEMV_TILE_WAVES, true};
      return best;
    }
  }
  // nothing fits: the largest items, waves looping over them
  const int S = std::min(64, (256 / nb) & (paired ? ~1 : ~0));
  return Shape{true, std::max(S, paired ? 2 : 1), 4, GEMV_TILE_WAVES};
}

size_t lds_bytes(const GemvArgs& a, const Shape& sh, int prologue) {
  const int attn = prologue == PRO_ATTN_EVEN ? 1 : prologue == PRO_ATTN_ONE ? 2 : 0;
  return static_cast<size_t>(lds_plan(a.nb, sh.S, sh.tile, attn, sh.grp ? 1 : sh.NW).words) * 4;
}

template <int PRO, int EPI, bool TILE, int WT, bool GRP = false>
int grid_for(int n_items, const Shape& sh, int n_cu, size_t lds) {
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &occ, reinterpret_cast<const void*>(k_gemv<PRO, EPI, TILE, WT, GRP>), 64 * sh.NW, lds) != hipSuccess ||
      occ < 1)
    occ = 1;
  // one resident round of work groups: more would queue behind the first
  const int per_group = GRP ? 1 : sh.NW;
  return std::min((n_items + per_group - 1) / per_group, n_cu * occ);
}

// Items of the launch; in region mode also each region's first item.
int n_items_of(GemvArgs& a, const Shape& sh) {
  if (a.pair) return items_for(a, sh.S);
  int n = 0;
  for (int i = 0; i < a.nreg; ++i) {
    a.reg[i].row0 = n;
    n += (a.reg[i].rows + sh.S - 1) / sh.S;
  }
  return n;
}

// PRO_ATTN_ONE: query heads per work group (1, 2 or 4, one kv head's) so
// that the work groups of every XCD (at least grid / 8 of them) cover every
// head; 0 when they cannot.
int attn_one_hpw(int grid, int nb) {
  const int nh = nb * QK_K / 64, per_xcd = grid / 8;
  for (int hpw = 1; hpw <= 4; hpw *= 2)
    if (per_xcd * hpw >= nh) return hpw;
  return 0;
}

template <int PRO, int EPI, bool TILE, int WT, bool GRP = false>
hipError_t launch_one(const GemvArgs& a0, int n_items, const Shape& sh, int n_cu, size_t lds, hipStream_t s) {
  if (TILE && sh.NW != GEMV_TILE_WAVES) return hipErrorInvalidValue;  // the kernel's launch bound
  if (GRP && (sh.S * a0.nb > 256 * sh.KB || sh.S > 64)) return hipErrorInvalidValue;
  const int grid = grid_for<PRO, EPI, TILE, WT, GRP>(n_items, sh, n_cu, lds);
  GemvArgs a = a0;
  if constexpr (PRO == PRO_ATTN_ONE) {
    // every work group resident at once (grid_for: one round), 4 waves
    a.attn_hpw = attn_one_hpw(grid, a.nb);
    if (!a.attn_hpw || sh.NW != 4 || !a.xrec || !a.epoch || !a.xcc || !a.err) return hipErrorNotSupported;
  }
  // the argmax partials: one per wave of the grid, as many as the caller sized
  if (EPI == EPI_LOGITS && grid * sh.NW != a.argmax_parts) return hipErrorInvalidValue;
  if (grid <= 0) return hipSuccess;
  launch_kernel(k_gemv<PRO, EPI, TILE, WT, GRP>, dim3(grid), dim3(64 * sh.NW), lds, s, a, n_items, sh.S, sh.KB);
  return hipGetLastError();
}

// the weight types of the launch's regions
int weight_kind(const GemvArgs& a) {
  bool q4 = false, q6 = false;
  for (int i = 0; i < a.nreg; ++i) (a.reg[i].w.type == MCPM_TYPE_Q4_K ? q4 : q6) = true;
  return q4 && q6 ? WT_MIX : q4 ? WT_Q4 : WT_Q6;
}

template <int PRO, int EPI>
hipError_t launch_pe(const GemvArgs& a0, const Shape& sh, int n_cu, hipStream_t s) {
  GemvArgs a = a0;
  const int n_items = n_items_of(a, sh);
  const size_t lds = lds_bytes(a, sh, PRO);
  const int wt = weight_kind(a);
  if constexpr (EPI == EPI_RESID || EPI == EPI_STORE) {
    if (sh.grp && wt == WT_Q4) return launch_one<PRO, EPI, true, WT_Q4, true>(a, n_items, sh, n_cu, lds, s);
    if (sh.grp && wt == WT_Q6) return launch_one<PRO, EPI, true, WT_Q6, true>(a, n_items, sh, n_cu, lds, s);
  }
  if (sh.grp) return hipErrorInvalidValue;
#define MCPM_WT(TT, WW) \
  if (sh.tile == TT && wt == WW) return launch_one<PRO, EPI, TT, WW>(a, n_items, sh, n_cu, lds, s);
  MCPM_WT(true, WT_Q4) MCPM_WT(true, WT_Q6) MCPM_WT(false, WT_Q4) MCPM_WT(false, WT_Q6)
  if constexpr (EPI == EPI_QKV || EPI == EPI_STORE) {  // the QKV regions (fused, or the per-op entry)
    MCPM_WT(true, WT_MIX) MCPM_WT(false, WT_MIX)
  }
#undef MCPM_WT
  return hipErrorInvalidValue;
}

}  // namespace

int gemv_attn_one_hpw(const GemvArgs& a0, int n_cu) {
  GemvArgs a = a0;
  const Shape sh = pick_shape(a, PRO_ATTN_ONE, EPI_RESID, n_cu);
  const int n_items = n_items_of(a, sh);
  const size_t lds = lds_bytes(a, sh, PRO_ATTN_ONE);
  int grid = 0;
  if (sh.grp && weight_kind(a) == WT_Q4) grid = grid_for<PRO_ATTN_ONE, EPI_RESID, true, WT_Q4, true>(n_items, sh, n_cu, lds);
  else if (sh.grp && weight_kind(a) == WT_Q6) grid = grid_for<PRO_ATTN_ONE, EPI_RESID, true, WT_Q6, true>(n_items, sh, n_cu, lds);
  else return 0;
  return sh.NW == 4 ? attn_one_hpw(grid, a.nb) : 0;
}

int gemv_grid(const GemvArgs& a0, int n_cu) {
  // number of argmax partials the LM-head launch (PRO_NORM_EVEN, EPI_LOGITS)
  // writes: one per wave
  GemvArgs a = a0;
  a.nreg = 1;
  a.reg[0].rows = a.total_rows;
  const Shape sh = pick_shape(a, PRO_NORM_EVEN, EPI_LOGITS, n_cu);
  const int n_items = n_items_of(a, sh);
  const size_t lds = lds_bytes(a, sh, PRO_NORM_EVEN);
  const bool q4 = weight_kind(a) == WT_Q4;  // a.reg[0].w must be the head's weights
  constexpr int P = PRO_NORM_EVEN, E = EPI_LOGITS;
  const int grid = sh.tile ? (q4 ? grid_for<P, E, true, WT_Q4>(n_items, sh, n_cu, lds)
                                 : grid_for<P, E, true, WT_Q6>(n_items, sh, n_cu, lds))
                           : (q4 ? grid_for<P, E, false, WT_Q4>(n_items, sh, n_cu, lds)
                                 : grid_for<P, E, false, WT_Q6>(n_items, sh, n_cu, lds));
  return grid * sh.NW;
}

hipError_t launch_ffn_fused(const GemvArgs& gu0, const GemvArgs& dn0, int n_cu, const GridSync& gs, hipStream_t s) {
  if (gu0.nb <= 0 || gu0.nb > MAX_NB || dn0.nb <= 0 || dn0.nb > MAX_NB || !gu0.pair || gu0.reg[0].w.type != MCPM_TYPE_Q4_K ||
      gu0.reg[1].w.type != MCPM_TYPE_Q4_K || dn0.nreg != 1)
    return hipErrorInvalidValue;
  GemvArgs gu = gu0, dn = dn0;
  const Shape sg = pick_shape(gu, PRO_NORM_AWAY, EPI_SWIGLU, n_cu);
  const Shape sd = pick_shape(dn, PRO_QUANT_AWAY, EPI_RESID, n_cu);
  if (!sg.tile || sg.grp || !sd.tile) return hipErrorNotSupported;  // the fused kernel runs TILE phases only
  const int gi = n_items_of(gu, sg), di = n_items_of(dn, sd);
  const int gg = (gi + GEMV_TILE_WAVES - 1) / GEMV_TILE_WAVES, dg = sd.grp ? di : (di + GEMV_TILE_WAVES - 1) / GEMV_TILE_WAVES;
  // one work group per CU, all resident; always n_cu of them, so that every
  // launch on the same barrier state counts the same arrivals per XCD
  if (gg > n_cu || dg > n_cu) return hipErrorNotSupported;
  const int grid = n_cu;
  const size_t lds = std::max(lds_bytes(gu, sg, PRO_NORM_AWAY), lds_bytes(dn, sd, PRO_QUANT_AWAY));
  const bool q6 = dn.reg[0].w.type == MCPM_TYPE_Q6_K;
#define MCPM_FUSED(WT, G)                                                                                            \
  launch_kernel(k_ffn_fused<WT, G>, dim3(grid), dim3(64 * GEMV_TILE_WAVES), lds, s, gu, gi, sg.S, sg.KB, gg, dn, di, \
                sd.S, sd.KB, dg, gs)
  if (q6 && sd.grp) MCPM_FUSED(WT_Q6, true);
  else if (q6) MCPM_FUSED(WT_Q6, false);
  else if (sd.grp) MCPM_FUSED(WT_Q4, true);
  else MCPM_FUSED(WT_Q4, false);
#undef MCPM_FUSED
  return hipGetLastError();
}

hipError_t launch_gemv(const GemvArgs& a, int prologue, int epilogue, int n_cu, hipStream_t s) {
  if (a.nb <= 0 || a.nb > MAX_NB) return hipErrorInvalidValue;
  if (prologue == PRO_ATTN_EVEN && (a.nb > ATTN_MAX_NB || a.head_dim <= 0 || a.head_dim % ATTN_VALS))
    return hipErrorInvalidValue;
  // PRO_ATTN_ONE: head_dim 64, four query heads per kv head (nb*256 = 4 * kvd)
  if (prologue == PRO_ATTN_ONE && (a.nb > ATTN_MAX_NB || a.head_dim != 64 || a.kvd * 4 != a.nb * QK_K ||
                                   !a.k_cache || !a.v_cache || !a.state || !a.x))
    return hipErrorInvalidValue;
  if (a.pair && a.reg[0].w.type != a.reg[1].w.type) return hipErrorInvalidValue;
  GemvArgs b = a;
  if (!b.pair && epilogue == EPI_LOGITS) {
    b.nreg = 1;
    b.reg[0].rows = b.total_rows;
  }
  const Shape sh = pick_shape(b, prologue, epilogue, n_cu);
#define MCPM_PE(PP, EE) \
  if (prologue == PP && epilogue == EE) return launch_pe<PP, EE>(b, sh, n_cu, s);
  MCPM_PE(PRO_Q8K, EPI_STORE)
  MCPM_PE(PRO_Q8K, EPI_RESID)
  MCPM_PE(PRO_QUANT_EVEN, EPI_STORE)
  MCPM_PE(PRO_QUANT_EVEN, EPI_RESID)
  MCPM_PE(PRO_ATTN_EVEN, EPI_RESID)
  MCPM_PE(PRO_ATTN_ONE, EPI_RESID)
  MCPM_PE(PRO_QUANT_AWAY, EPI_RESID)
  MCPM_PE(PRO_NORM_AWAY, EPI_QKV)
  MCPM_PE(PRO_NORM_AWAY, EPI_SWIGLU)
  MCPM_PE(PRO_NORM_EVEN, EPI_LOGITS)
  MCPM_PE(PRO_NORM_EVEN, EPI_STORE)
#undef MCPM_PE
  return hipErrorInvalidValue;
}

hipError_t launch_qkv_attn(const GemvArgs& q0, const AttnArgs& at, int n_cu, const GridSync& gs, hipStream_t s) {
  if (q0.nb <= 0 || q0.nb > MAX_NB || q0.nreg != 3 || q0.pair || at.head_dim <= 0 || at.head_dim > 128 ||
      at.head_dim % 4 || at.n_kv_heads <= 0 || at.n_heads % at.n_kv_heads ||
      at.n_heads / at.n_kv_heads > ATTN_MAX_GROUP || at.head_dim != q0.head_dim)
    return hipErrorInvalidValue;
  // the rows at pos are read again through 32-bit buffer offsets
  if (static_cast<size_t>(at.max_chunks) * ATTN_CHUNK * at.n_kv_heads * at.head_dim * sizeof(float) >= (size_t{1} << 31))
    return hipErrorNotSupported;
  GemvArgs qa = q0;
  const Shape sh = pick_shape(qa, PRO_NORM_AWAY, EPI_QKV, n_cu);
  if (!sh.tile || sh.grp) return hipErrorNotSupported;  // the fused kernel runs a TILE phase
  const int qi = n_items_of(qa, sh);
  const int qg = (qi + GEMV_TILE_WAVES - 1) / GEMV_TILE_WAVES;
  // one work group per CU, all resident; always n_cu of them, so that every
  // launch on the same barrier state counts the same arrivals per XCD
  if (qg > n_cu) return hipErrorNotSupported;
  const int grid = n_cu;
  const bool h64 = at.head_dim <= 64;
  const size_t lds =
      std::max(lds_bytes(qa, sh, PRO_NORM_AWAY), h64 ? AttnLds<64>::bytes : AttnLds<128>::bytes);
  const int wt = weight_kind(qa);
#define MCPM_QA(WW, HH)                                                                                    \
  if (wt == WW && (HH == 64) == h64) {                                                                     \
    if (lds > 65536) {                                                                                     \
      const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(k_qkv_attn<WW, HH>),       \
                                                  hipFuncAttributeMaxDynamicSharedMemorySize,              \
                                                  static_cast<int>(lds));                                  \
      if (attr != hipSuccess) return attr;                                                                 \
    }                                                                                                      \
    launch_kernel(k_qkv_attn<WW, HH>, dim3(grid), dim3(64 * GEMV_TILE_WAVES), lds, s, qa, qi, sh.S, sh.KB, \
                  qg, at, gs);                                                                             \
    return hipGetLastError();                                                                              \
  }
  MCPM_QA(WT_Q4, 64) MCPM_QA(WT_Q6, 64) MCPM_QA(WT_MIX, 64)
  MCPM_QA(WT_Q4, 128) MCPM_QA(WT_Q6, 128) MCPM_QA(WT_MIX, 128)
#undef MCPM_QA
  return hipErrorInvalidValue;
}

}  // namespace mcpm
