// mcpm_attn.h -- the decode attention's device code, shared by its own
// kernel (mcpm_kernels.hip) and the QKV + attention kernel (mcpm_gemv.hip).
#pragma once

#include <algorithm>

#include "mcpm_device.h"

namespace mcpm {

// ------------------------------------------------------------- attention ---
// A work group of 256 threads per (kv head, split); a split takes consecutive
// chunks of ATTN_CHUNK positions, and the group's query heads (n_heads /
// n_kv_heads, at most 8) share each K and V row.  Per chunk c and head h:
//   s_t = (fma chain over i of q_i*k_ti) * scale          (thread <-> (h, t))
//   m_c = max(-1e9, s_t); e_t = exp(s_t - m_c); z_c = pairwise tree over 64 slots
//   o_c[i] = fma chain over t of e_t*v_ti                  (thread <-> (h, i))
// and over the chunks, in order:
//   m = max m_c; f_c = exp(m_c - m); Z = fma(z_c, f_c, Z); O_i = fma(o_c[i], f_c, O_i)
//   out_i = O_i / Z
// A split takes ceil(nch/64) consecutive chunks (at most ATTN_CPW), keeping
// o_c in registers, so a kv head has at most 64 splits (up to 64*ATTN_CPW
// chunks): one chunk per work group up to 4096 positions.  Every split
// writes its chunks' partials; the combine over the chunks runs in the
// consumer (the O-projection's prologue, or k_attn_combine), after the
// kernel boundary, so no split waits for another.
// Partials (AttnPart): o_c at o[(h*max_chunks + c)*head_dim + i], (m_c, z_c)
// at mz[h*max_chunks + c].  Every load of a chunk's K and V rows is issued at
// once, one chunk ahead, and the rows are staged through LDS.
constexpr int ATTN_MAX_SPLITS = 64;

__host__ __device__ inline int attn_chunks_per_split(int nch) {
  const int c = (nch + ATTN_MAX_SPLITS - 1) / ATTN_MAX_SPLITS;
  return c < 1 ? 1 : (c > ATTN_CPW ? ATTN_CPW : c);
}
__host__ __device__ inline int attn_splits(int nch) {
  const int cps = attn_chunks_per_split(nch);
  return (nch + cps - 1) / cps;
}
// The split count is not monotonic in the chunk count (64 chunks take 64
// splits, 66 take 33): a launch covers the most any count in [lo, hi] needs.
inline int attn_max_splits(int lo, int hi) {
  int m = 1;
  for (int n = std::max(lo, 1); n <= hi; ++n) m = std::max(m, attn_splits(n));
  return m;
}

// Maximum over the wave (order-free): lane moves within rows of 16, then
// across rows.
__device__ __forceinline__ float wave_max_fast(float v) {
  v = row16_max(v);
  v = fmaxf(v, lane_xor16(v));
  v = fmaxf(v, lane_xor32(v));
  return v;
}

template <int NV>
struct AttnRegs {
  f32x4 k[NV];
  f32x4 v[NV];
};

// K and V rows of chunk c into registers: thread slot f = tid + 256u holds
// float4 f%r4 of row f/r4; slots past the chunk read its last element and
// positions past T read row T-1 (in bounds, unused).  SKIP_LAST: slots of
// row T-1 are not loaded.  That row is being written by other work groups of
// the same launch: a plain load issued before the writers are done would
// leave a stale line in this XCD's L2, which later loads of the launch,
// coherent ones included, could then hit; attn_reload_last_row fills those
// slots once the writers are done.
// tid: the thread's index in its group of 256 (the work group's by default).
template <int NV, bool SKIP_LAST = false>
__device__ __forceinline__ void attn_load_chunk(AttnRegs<NV>& R, const float* __restrict__ kc,
                                                const float* __restrict__ vc, int c, int T, int kvd,
                                                size_t head_off, int r4, int nf4,
                                                int tid = static_cast<int>(threadIdx.x)) {
#pragma unroll
  for (int u = 0; u < NV; ++u) {
    const int f = min(tid + 256 * u, nf4 - 1);
    const int j = f / r4, c4 = f - j * r4;
    const int t = min(c * ATTN_CHUNK + j, T - 1);
    const size_t o = static_cast<size_t>(t) * kvd + head_off + c4 * 4;
    if (!SKIP_LAST || t != T - 1) {
      R.k[u] = *reinterpret_cast<const f32x4*>(kc + o);
      R.v[u] = *reinterpret_cast<const f32x4*>(vc + o);
    }
  }
}

// One token on one chunk staged in LDS (K rows in sK with stride HDM + 4, V
// rows in sV, the token's group of queries in sQ): scores and softmax terms
// (wave <-> head, lane <-> position) into sE and mz[hh] = (m_c, z_c), a
// barrier, then the weighted V sums, thread (head, dim) oi = tid + 256u into
// o[u].  Positions at or past T take no part.  tid: the thread's index in its
// group of 256 (the work group's by default); with WL (a wave-level ordering
// between the two phases) several groups may run chunks side by side.
template <int HDM, int OPT, bool WL = false>
__device__ __forceinline__ void attn_token_chunk(const float* sK, const float* sV, const float* sQ, float* sE,
                                                 float2* mz, int c, int T, int group, int hd, int gh, float scale,
                                                 float (&o)[OPT], int tid = static_cast<int>(threadIdx.x)) {
  constexpr int KS = HDM + 4;
  const int lane = tid & 63, wave = tid >> 6;
  for (int hh = wave; hh < group; hh += 4) {
    const float* qh = &sQ[hh * HDM];
    const float* kt = &sK[lane * KS];
    float dot = 0.0f;
#pragma unroll 4
    for (int i = 0; i < hd; i += 4) {
      const f32x4 k4 = *reinterpret_cast<const f32x4*>(kt + i);
      const f32x4 q4 = *reinterpret_cast<const f32x4*>(qh + i);
      dot = __builtin_fmaf(q4.x, k4.x, dot);
      dot = __builtin_fmaf(q4.y, k4.y, dot);
      dot = __builtin_fmaf(q4.z, k4.z, dot);
      dot = __builtin_fmaf(q4.w, k4.w, dot);
    }
    const bool present = c * ATTN_CHUNK + lane < T;
    const float sv = present ? dot * scale : -1e9f;
    const float mc = fmaxf(wave_max_fast(sv), -1e9f);
    const float e = present ? exp_f32(sv - mc) : 0.0f;
    const float z = wave_tree_sum_fast(e);
    sE[hh * ATTN_CHUNK + lane] = e;
    if (lane == 0) mz[hh] = make_float2(mc, z);
  }
  // WL (head_dim 64): head hh's weighted sums run on the wave that formed
  // its softmax terms, so a wave-level ordering suffices
  if constexpr (WL) wave_sync();
  else __syncthreads();
  const int nt = min(ATTN_CHUNK, T - c * ATTN_CHUNK);
#pragma unroll
  for (int u = 0; u < OPT; ++u) {
    const int oi = tid + 256 * u;
    float acc = 0.0f;
    if (oi < gh) {
      const int hh = oi / hd, i = oi - hh * hd;
      const float* eh = &sE[hh * ATTN_CHUNK];
#pragma unroll 8
      for (int j = 0; j < nt; ++j) acc = __builtin_fmaf(eh[j], sV[j * HDM + i], acc);
    }
    o[u] = acc;
  }
}

// K and V elements of row T-1 among chunk c's register slots, read again
// through the coherence point: that row was written by other work groups of
// the same launch, after the slots were first loaded.
template <int NV>
__device__ __forceinline__ void attn_reload_last_row(AttnRegs<NV>& R, const float* kc, const float* vc, int c, int T,
                                                     int kvd, size_t head_off, int r4, int nf4) {
#pragma unroll
  for (int u = 0; u < NV; ++u) {
    const int f = min(static_cast<int>(threadIdx.x) + 256 * u, nf4 - 1);
    const int j = f / r4, c4 = f - j * r4;
    if (min(c * ATTN_CHUNK + j, T - 1) == T - 1) {
      const uint32_t o = static_cast<uint32_t>((static_cast<size_t>(T - 1) * kvd + head_off + c4 * 4) * 4);
      R.k[u] = ld_coh4(kc, o);
      R.v[u] = ld_coh4(vc, o);
    }
  }
}

// LDS of one split: K rows (stride HDM + 4), V rows, the group's queries,
// softmax terms and the chunks' (m_c, z_c).
template <int HDM>
struct AttnLds {
  static constexpr int K = ATTN_CHUNK * (HDM + 4), V = ATTN_CHUNK * HDM, Q = ATTN_MAX_GROUP * HDM,
                       E = ATTN_MAX_GROUP * ATTN_CHUNK, MZ = ATTN_CPW * ATTN_MAX_GROUP;
  static constexpr size_t bytes = (K + V + Q + E) * sizeof(float) + MZ * sizeof(float2);
  float* sK;
  float* sV;
  float* sQ;
  float* sE;
  float2* sMZ;
  __device__ __forceinline__ explicit AttnLds(float* base)
      : sK(base), sV(base + K), sQ(base + K + V), sE(base + K + V + Q), sMZ(reinterpret_cast<float2*>(base + K + V + Q + E)) {}
};

// Chunks c0 .. c0+n-1 (n <= ATTN_CPW) of kv head kvh at context T: o_c of
// thread (head, dim) oi = tid + 256u into oc[u][cc], (m_c, z_c) of head hh
// into S.sMZ[cc*ATTN_MAX_GROUP + hh] (written by lane 0 of wave hh % 4).
// COH: q and the K and V rows at T-1 were written by other work groups of the
// same launch and are read through the coherence point.  pre: chunk c0 is
// already in R (attn_load_chunk by the caller).
template <int HDM, bool COH, bool WL>
__device__ __forceinline__ void attn_chunks(const float* __restrict__ q, const float* __restrict__ kc,
                                            const float* __restrict__ vc, int T, int kvh, int c0, int n, int group,
                                            int hd, int kvd, const AttnLds<HDM>& S, AttnRegs<HDM / 16>& R, bool pre,
                                            float (&oc)[ATTN_MAX_GROUP * HDM / 256][ATTN_CPW]) {
  constexpr int NV = HDM / 16;                      // float4 of a chunk's K (or V) per thread, at most
  constexpr int OPT = ATTN_MAX_GROUP * HDM / 256;   // outputs per thread, at most
  constexpr int NQ = ATTN_MAX_GROUP * HDM / 256;    // query values per thread, at most
  constexpr int KS = HDM + 4;                       // LDS row stride of K
  float* sK = S.sK;
  float* sV = S.sV;
  float* sQ = S.sQ;
  float* sE = S.sE;
  float2* sMZ = S.sMZ;
  const int tid = threadIdx.x;
  const int nch = (T + ATTN_CHUNK - 1) / ATTN_CHUNK;
  const int r4 = hd / 4;              // float4 per K/V row
  const int nf4 = ATTN_CHUNK * r4;    // float4 per chunk
  const int gh = group * hd;          // outputs of the work group
  const float scale = 1.0f / sqrtf(static_cast<float>(hd));
  const size_t head_off = static_cast<size_t>(kvh) * hd;

  if (!pre) attn_load_chunk<NV>(R, kc, vc, c0, T, kvd, head_off, r4, nf4);
  {
    const float* qg = q + static_cast<size_t>(kvh) * gh;
    float qv[NQ];
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const float* p = qg + min(tid + 256 * u, gh - 1);
      if constexpr (COH) qv[u] = ld_coh(p);
      else qv[u] = *p;
    }
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const int i = tid + 256 * u;
      if (i < gh) sQ[(i / hd) * HDM + i % hd] = qv[u];
    }
  }

#pragma clang loop unroll(full)
  for (int cc = 0; cc < ATTN_CPW; ++cc) {
    if (cc < n) {
      const int c = c0 + cc;
      if constexpr (COH) {
        if (c == nch - 1) attn_reload_last_row<NV>(R, kc, vc, c, T, kvd, head_off, r4, nf4);
      }
      __syncthreads();  // readers of the previous chunk are done
      // slots past the chunk rewrite its last element with the same value
#pragma unroll
      for (int u = 0; u < NV; ++u) {
        const int f = min(tid + 256 * u, nf4 - 1);
        const int j = f / r4, c4 = f - j * r4;
        *reinterpret_cast<f32x4*>(&sK[j * KS + c4 * 4]) = R.k[u];
        *reinterpret_cast<f32x4*>(&sV[j * HDM + c4 * 4]) = R.v[u];
      }
      if (cc + 1 < n) attn_load_chunk<NV>(R, kc, vc, c + 1, T, kvd, head_off, r4, nf4);
      __syncthreads();
      float o[OPT];
      attn_token_chunk<HDM, OPT, WL>(sK, sV, sQ, sE, sMZ + cc * ATTN_MAX_GROUP, c, T, group, hd, gh, scale, o);
#pragma unroll
      for (int u = 0; u < OPT; ++u) oc[u][cc] = o[u];
    }
  }
}

// Split `split` of kv head kvh at context T: its chunks' partials (the work
// of one k_attention work group).  COH and pre as for attn_chunks.
template <int HDM, bool COH, bool WL = false>
__device__ __forceinline__ void attn_split(const float* __restrict__ q, const float* __restrict__ kc,
                                           const float* __restrict__ vc, int T, int kvh, int split, int n_heads,
                                           int n_kv_heads, int hd, int max_chunks, float* __restrict__ part_o,
                                           float2* __restrict__ part_mz, const AttnLds<HDM>& S,
                                           AttnRegs<HDM / 16>& R, bool pre) {
  constexpr int OPT = ATTN_MAX_GROUP * HDM / 256;   // outputs per thread, at most
  const int tid = threadIdx.x;
  const int nch = (T + ATTN_CHUNK - 1) / ATTN_CHUNK;
  const int cps = attn_chunks_per_split(nch);
  const int nsplit = attn_splits(nch);
  if (split >= nsplit) return;
  const int c0 = split * cps, n = min(cps, nch - c0);
  const int group = n_heads / n_kv_heads;
  const int gh = group * hd;          // outputs of the work group
  float2* sMZ = S.sMZ;

  float oc[OPT][ATTN_CPW];
  attn_chunks<HDM, COH, WL>(q, kc, vc, T, kvh, c0, n, group, hd, n_kv_heads * hd, S, R, pre, oc);

  // this split's chunks to the partials
#pragma unroll
  for (int u = 0; u < OPT; ++u) {
    const int oi = tid + 256 * u;
    if (oi < gh) {
      const int hh = oi / hd, i = oi - hh * hd;
      float* ph = part_o + (static_cast<size_t>(kvh * group + hh) * max_chunks + c0) * hd + i;
#pragma unroll
      for (int cc = 0; cc < ATTN_CPW; ++cc)
        if (cc < n) ph[static_cast<size_t>(cc) * hd] = oc[u][cc];
    }
  }
  if constexpr (WL) {
    // (m_c, z_c) stored by lane 0 of the wave that wrote them (heads wave,
    // wave + 4)
    if ((tid & 63) == 0) {
      for (int hh = tid >> 6; hh < group; hh += 4)
        for (int cc = 0; cc < n; ++cc)
          part_mz[static_cast<size_t>(kvh * group + hh) * max_chunks + c0 + cc] = sMZ[cc * ATTN_MAX_GROUP + hh];
    }
  } else if (tid < ATTN_CPW * ATTN_MAX_GROUP) {
    const int cc = tid / ATTN_MAX_GROUP, hh = tid % ATTN_MAX_GROUP;
    if (cc < n && hh < group) part_mz[static_cast<size_t>(kvh * group + hh) * max_chunks + c0 + cc] = sMZ[cc * ATTN_MAX_GROUP + hh];
  }
}

}  // namespace mcpm
