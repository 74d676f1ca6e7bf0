// mcpm_persist.hip -- every decoder layer of one token in one launch
// (src/model.cpp:171-226, the layer loop of MiniCPM5Engine::forward).
//
// The per-token kernel sequence runs five launches per layer; each starts
// by waiting for the previous launch's last wave and then for its own first
// weights.  Here one work group per CU (b on XCD b % 8) runs all layers:
//   E  the token's embedding values of this work group's rows of x
//   Q  RMSNorm + Q8_K (ties away) of x; the q, k and v rows of kv head
//      h = b % 8 (so head h's rows are computed on XCD h); RoPE; K and V
//      rows at pos into the cache
//   A  attention of kv head h: chunk c of 64 positions on work group
//      (h, c mod W); work group (h, W-1), which has no chunk below W chunks,
//      combines the chunks' partials in chunk order and quantizes the head
//      group's output ties-even (Q8_K blocks); with one chunk its owner
//      finishes the head itself
//   O  O projection of this work group's rows of x, residual add
//   G  RMSNorm + Q8_K (ties away); gate and up rows of its FFN pairs; SwiGLU
//   D  Q8_K (ties away) of h; down projection of its rows of x; residual add
// The arithmetic of every phase is that of the per-token kernels (lane sums
// of src/ops/ops_avx2.cpp:153-276, the float chain over blocks, the chunked
// softmax), so results are bit-identical to them.
//
// Hand-offs.  A phase's outputs go to the next phase's work groups as
// records of (value bits, tag), stored and loaded as 64-bit atomics at agent
// scope: a consumer spins until every record it needs carries the tag of the
// current (launch, layer); no barrier counter and no fence.  Records are
// reused by every layer and launch; the tag tells them apart, and no work
// group can be more than one phase ahead of another (each phase needs every
// work group's output of the one before), so a record is never rewritten
// while a reader still waits for its previous value.
//
// Weights.  Each work group's share of a layer is a contiguous slab (built
// once from the weight planes), in four regions: QKV, O, gate/up, down.  A
// region is copied into LDS (direct-to-LDS loads, 1 KiB per wave
// instruction) after its previous use, during the hand-off wait of a phase
// before the one that reads it: O at Q; the next layer's QKV, this layer's
// gate/up and down at O, where every other phase's wait is an all-to-all
// wait but O's runs beside the attention (on the work groups that combine
// attention chunks gate/up at A, while they wait for the chunks' partials,
// the rest at G; on the owner of a single chunk, which reaches O last,
// gate/up at O and the rest at G).  The wait ends with every copy landed.  The chunk owners' K and V rows go into the gate/up
// region at the previous layer's D (where that region holds them; the
// combining work group's into the down region at Q), the attention's
// staging.
//
// Every wait is bounded: past spin_limit, or once another work group has
// given up, the work group sets the error word and returns.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "mcpm_attn.h"
#include "mcpm_device.h"
#include "mcpm_persist.h"

namespace mcpm {

static_assert(PD_ATTN_LDS == static_cast<int>(AttnLds<64>::bytes), "attention staging size");

namespace {

// The fixed plan's fields as compile-time constants for the instance built
// for it (FS); the other instance reads the launch's plan.  The layer count
// and the chunk count always come from the launch (a.s).
__device__ constexpr PdShape kPdFixed = pd_fixed_plan();
template <bool FS>
__device__ __forceinline__ const PdShape& pd_s(const PdArgs& a) {
  if constexpr (FS) return kPdFixed;
  else return a.s;
}

typedef short pd_i16x2 __attribute__((ext_vector_type(2)));
constexpr int CHAIN_BATCH_PD = 12;  // chain entries read per LDS round trip

__device__ __forceinline__ uint64_t rec_ld(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void rec_st(uint64_t* p, uint32_t v, uint32_t tag) {
  __hip_atomic_store(p, (static_cast<uint64_t>(tag) << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void rec_stf(uint64_t* p, float v, uint32_t tag) { rec_st(p, __float_as_uint(v), tag); }
// A record read only on its writer's XCD (a kv head's q/k/v rows, its
// chunks' partials): in the XCD-local instance (XL) a workgroup-scope
// store, which leaves it in that XCD's L2 (the vector L1 writes through),
// where the readers' agent-scope loads find it; else an agent-scope store.
// The scope is a template parameter: a run-time choice costs code in a
// kernel whose loop fills the instruction cache.
template <bool XL>
__device__ __forceinline__ void rec_stf_xcd(uint64_t* p, float v, uint32_t tag) {
  const uint64_t r = (static_cast<uint64_t>(tag) << 32) | __float_as_uint(v);
  if constexpr (XL) __hip_atomic_store(p, r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  else __hip_atomic_store(p, r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_u32c(const unsigned* p) {
  return __hip_atomic_load(const_cast<unsigned*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_u32c(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int pd_dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}
__device__ __forceinline__ int pd_dot2(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot2(__builtin_bit_cast(pd_i16x2, a), __builtin_bit_cast(pd_i16x2, b), c, false);
}
__device__ __forceinline__ uint32_t pd_byte_pair(uint32_t w, int k) {
  return __builtin_amdgcn_perm(0u, w, 0x0c000c00u | (static_cast<uint32_t>(k + 1) << 16) | static_cast<uint32_t>(k));
}
__device__ __forceinline__ int pd_mad24(int a, int b, int c) { return __mul24(a, b) + c; }
__device__ __forceinline__ uint32_t comp(const u32x4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Work-group barrier ordering LDS only: it does not wait for the waves'
// vector memory operations, so weight copies stay in flight across it.
__device__ __forceinline__ void pd_bar() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Any thread's v, on every thread, with one barrier: each wave's vote in one
// of two slot sets (by call parity, it counts the work group's calls), so a
// set is rewritten only after every thread has read it.
__device__ __forceinline__ bool pd_any(bool v, uint32_t* slots, uint32_t& it) {
  const bool w = __any(v);
  uint32_t* q = slots + 4 * (it & 1u);
  if ((threadIdx.x & 63) == 0) q[threadIdx.x >> 6] = w ? 1u : 0u;
  pd_bar();
  ++it;
  return (q[0] | q[1] | q[2] | q[3]) != 0u;
}

// The work group's RMS factor 1/sqrt(sum/dim + eps) from thread t's partial
// p (t < 256): the 256-slot tree of block_rms_1sync, with an LDS-only
// barrier.
__device__ __forceinline__ float pd_rms(float p, int dim, float eps, float* s_red) {
  const int tid = static_cast<int>(threadIdx.x), lane = tid & 63;
  s_red[tid] = p;
  pd_bar();
  float v = (s_red[lane] + s_red[lane + 128]) + (s_red[lane + 64] + s_red[lane + 192]);
  v = wave_tree_sum_fast(v);
  v = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
  return 1.0f / sqrtf(v / static_cast<float>(dim) + eps);
}

// A region of a (layer, work group) slab into LDS: 1 KiB per wave
// instruction (global_load_lds_dwordx4: lane i's 16 bytes to M0 + 16i), the
// 4 waves taking every fourth KiB.  bytes is a multiple of 1 KiB.  Issued as
// assembly, so the compiler inserts no wait for it (it cannot prove that
// later LDS accesses miss the region, and would wait for the copy at the
// next one): the data is there once the issuing waves have waited for their
// vector memory counter, which the hand-off wait the copy is issued before
// does before its barrier, and the region is first read after that.
__device__ __forceinline__ void pd_copy(const uint8_t* src, uint8_t* lds, int bytes) {
  const int wave = static_cast<int>(threadIdx.x >> 6), lane = static_cast<int>(threadIdx.x & 63);
  const uint32_t l0 = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t*)(lds)));
  for (int i = wave; i < (bytes >> 10); i += 4) {
    const uint8_t* g = src + (static_cast<size_t>(i) << 10) + lane * 16;
    const uint32_t m = __builtin_amdgcn_readfirstlane(l0 + (static_cast<uint32_t>(i) << 10));
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" : : "s"(m), "v"(g) : "m0", "memory");
  }
}

// K and V rows of chunk c (positions 64c .. 64c+63) of the kv head at
// head_off into the attention's staging (K rows at a stride of 68 floats, V
// rows at 64: AttnLds<64>) with direct-to-LDS loads, 17 + 16 wave
// instructions of 1 KiB: lane i of instruction n writes bytes 1024n + 16i,
// so its source is the row and column that land there (a K row's padding
// reads the dummy).  Rows at or past T-1 read the dummy too: row T-1 is
// written in this launch (it comes from the QKV phase's records) and later
// rows are outside the context.  Like pd_copy, the data is there once the
// issuing waves have waited for their vector memory counter.
__device__ __forceinline__ void pd_stage_chunk(const float* kc, const float* vc, int c, int T, int kvd,
                                               size_t head_off, const float* dummy, uint8_t* lds) {
  const int wave = static_cast<int>(threadIdx.x >> 6), lane = static_cast<int>(threadIdx.x & 63);
  const uint32_t l0 = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t*)(lds)));
  constexpr int KROW = (64 + 4) * 4, VROW = 64 * 4, KB = 64 * KROW / 1024, VB = 64 * VROW / 1024;
  for (int n = wave; n < KB + VB; n += 4) {
    const bool isk = n < KB;
    const int pos = ((isk ? n : n - KB) << 10) + lane * 16;  // byte offset within the K or V rows
    const int rb = isk ? KROW : VROW;
    const int row = pos / rb, cb = pos - row * rb, j = ATTN_CHUNK * c + row;
    const float* src = cb < VROW && j < T - 1
                           ? (isk ? kc : vc) + static_cast<size_t>(j) * kvd + head_off + (cb >> 2)
                           : dummy;
    const uint32_t m = __builtin_amdgcn_readfirstlane(l0 + static_cast<uint32_t>(n << 10));
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" : : "s"(m), "v"(src) : "m0", "memory");
  }
}

// ------------------------------------------------------------ hand-offs ---
// Waits (the whole work group) until record idx(k) of buf carries `tag` for
// every k < K of every thread (idx < 0: no record, value 0); values to v.
// Ends with the thread's vector memory operations complete and a barrier.
// false: a wait passed the spin limit or another work group gave up (the
// error word is set).
template <int K, class F>
__device__ __forceinline__ bool pd_poll(const PdArgs& a, const uint64_t* buf, uint32_t tag, F idx, uint32_t (&v)[K],
                                        uint32_t* misc, uint32_t& vit) {
  uint64_t r[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int i = idx(k);
    r[k] = i >= 0 ? rec_ld(buf + i) : (static_cast<uint64_t>(tag) << 32);
  }
  uint32_t spins = 0;
  for (;;) {
    uint32_t pend = 0;
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (static_cast<uint32_t>(r[k] >> 32) != tag) pend |= 1u << k;
    ++spins;
    if (threadIdx.x == 0 && (spins > a.spin_limit || ((spins & 63) == 0 && ld_u32c(a.err)))) {
      misc[0] = 1;
      st_u32c(a.err, 1u);
    }
    // vmcnt(0), expcnt and lgkmcnt left free: every load and copy this wave
    // issued is complete (the builtin, so the compiler knows it)
    __builtin_amdgcn_s_waitcnt(0x0f70);
    const bool any = pd_any(pend != 0, misc + 4, vit);
    if (misc[0]) return false;
    if (!any) break;
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (pend & (1u << k)) r[k] = rec_ld(buf + idx(k));
  }
#pragma unroll
  for (int k = 0; k < K; ++k) v[k] = static_cast<uint32_t>(r[k]);
  return true;
}

// One thread's wait for the records p[i] whose bit i is set in mask (the
// others are not read and give 0); values to v.  false past the spin limit.
template <int N>
__device__ __forceinline__ bool pd_wait_m(const uint64_t* const (&p)[N], uint32_t mask, uint32_t tag, uint32_t limit,
                                          uint32_t (&v)[N]) {
  uint64_t r[N];
#pragma unroll
  for (int i = 0; i < N; ++i) r[i] = (mask >> i) & 1u ? rec_ld(p[i]) : (static_cast<uint64_t>(tag) << 32);
  for (uint32_t s = 0;; ++s) {
    bool done = true;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (static_cast<uint32_t>(r[i] >> 32) != tag) {
        done = false;
        r[i] = rec_ld(p[i]);
      }
    }
    if (done) break;
    if (s > limit) return false;
  }
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = static_cast<uint32_t>(r[i]);
  return true;
}

// ------------------------------------------------------ Q8_K activations ---
// Block b of the scratch's Q8_K activations from a row of 16 lanes (lane j
// holding values 16j..16j+15): codes, d, bsums and the bsum pair sums (the
// layout the lane sums read).  Every lane of the row takes part (lane moves).
__device__ __forceinline__ void pd_store_xblock(uint32_t* S, const PdShape& s, int b, int j, u32x4 q, float d,
                                                int bs) {
  const int v = bs + dpp_i<DPP_XOR1>(bs);
  const uint32_t w = (static_cast<uint32_t>(v) & 0xffffu) | (static_cast<uint32_t>(dpp_i<DPP_XOR2>(v)) << 16);
  *reinterpret_cast<u32x4*>(S + s.s_xs + b * 68 + 4 * j) = q;
  S[s.s_xbs + b * 16 + j] = static_cast<uint32_t>(bs);
  if (j == 0) S[s.s_xd + b] = __float_as_uint(d);
  if ((j & 3) == 0) S[s.s_xbp + b * 4 + (j >> 2)] = w;
}

// -------------------------------------------------------- lane sums -------
// Half h = p of a Q4_K (row, block): the lane sums isum[m] for m = 4p..4p+3
// (lane m owns bytes 4m..4m+3 of every 32-byte chunk; quant dword 8j+m is
// in chunk 2j+p), by summation by parts over the running dots as in the
// per-token GEMV; p = 0 also forms the min sum.  Entry e: words 4p..4p+3 the
// sums, p = 0: words 8..10 d_x*d, d_x*dmin, minsum.
__device__ __forceinline__ void q4k_half(const uint8_t* w, int R, int blk, int row, int p, const uint32_t* xs,
                                         const uint32_t* xbp, float xd, uint32_t* e) {
  const u32x4* base = reinterpret_cast<const u32x4*>(w) + static_cast<size_t>(blk) * 9 * R + row;
  const u32x4 hdr = base[8 * R];
  u32x4 qv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) qv[j] = base[(2 * j + p) * R];
  const uint32_t s0 = hdr.y, s1 = hdr.z, s2 = hdr.w;
  const uint32_t sc_lo = s0 & 0x3f3f3f3fu;
  const uint32_t sc_hi = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
  int sc[8], cf[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    sc[k] = static_cast<int>(__builtin_amdgcn_ubfe(sc_lo, 8 * k, 8));
    sc[4 + k] = static_cast<int>(__builtin_amdgcn_ubfe(sc_hi, 8 * k, 8));
  }
#pragma unroll
  for (int k = 0; k < 7; ++k) cf[k] = sc[k] - sc[k + 1];
  cf[7] = sc[7];
  int P[4], is[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const u32x4 xe = *reinterpret_cast<const u32x4*>(xs + 16 * j + 4 * p);
    const u32x4 xo = *reinterpret_cast<const u32x4*>(xs + 16 * j + 8 + 4 * p);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const uint32_t q = comp(qv[j], m);
      P[m] = pd_dot4(q & 0x0f0f0f0fu, comp(xe, m), j == 0 ? 0 : P[m]);
      is[m] = j == 0 ? __mul24(cf[0], P[m]) : pd_mad24(cf[2 * j], P[m], is[m]);
      P[m] = pd_dot4((q >> 4) & 0x0f0f0f0fu, comp(xo, m), P[m]);
      is[m] = pd_mad24(cf[2 * j + 1], P[m], is[m]);
    }
  }
  *reinterpret_cast<u32x4*>(e + 4 * p) = u32x4{static_cast<uint32_t>(is[0]), static_cast<uint32_t>(is[1]),
                                               static_cast<uint32_t>(is[2]), static_cast<uint32_t>(is[3])};
  if (p == 0) {
    const uint32_t mn_lo = s1 & 0x3f3f3f3fu;
    const uint32_t mn_hi = ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u);
    const u32x4 bp = *reinterpret_cast<const u32x4*>(xbp);
    int v = pd_dot2(pd_byte_pair(mn_lo, 0), bp.x, 0);
    v = pd_dot2(pd_byte_pair(mn_lo, 2), bp.y, v);
    v = pd_dot2(pd_byte_pair(mn_hi, 0), bp.z, v);
    const int ms = pd_dot2(pd_byte_pair(mn_hi, 2), bp.w, v);
    const float ds = xd * fp16_to_fp32(static_cast<uint16_t>(hdr.x & 0xffffu));
    const float dm = xd * fp16_to_fp32(static_cast<uint16_t>(hdr.x >> 16));
    e[8] = __float_as_uint(ds);
    e[9] = __float_as_uint(dm);
    e[10] = static_cast<uint32_t>(ms);
  }
}

// Half p of a Q6_K (row, block): lane sums m = 4p..4p+3 (codes in [0, 63],
// the -32 applied through the bsums), as the per-token GEMV: for half h of
// the block, ql dwords 16h+m and 16h+8+m (chunks 4h+p and 4h+2+p), qh dword
// 8h+m (chunk 8+2h+p), activations 32h+8g+m, scale 8h+2g+p.
__device__ __forceinline__ void q6k_half(const uint8_t* w, int R, int nb, int blk, int row, int p,
                                         const uint32_t* xs, const uint32_t* xbs, float xd, uint32_t* e) {
  const u32x4* base = reinterpret_cast<const u32x4*>(w) + static_cast<size_t>(blk) * 13 * R + row;
  const u32x4 scv = base[12 * R];
  const uint32_t dword = reinterpret_cast<const uint32_t*>(w + 208 * R * nb)[blk * R + row];
  u32x4 a0[2], a1[2], hb[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    a0[h] = base[(4 * h + p) * R];
    a1[h] = base[(4 * h + 2 + p) * R];
    hb[h] = base[(8 + 2 * h + p) * R];
  }
  // term k = 4h+g has scale sc[8h+2g+p]: byte 2(g&1)+p of scale dword
  // 2h+(g>>1), taken with a bit offset that depends on the half p (no
  // lookup by a runtime index); by parts as the per-token GEMV
  int scp[8], cf[8];
#pragma unroll
  for (int k = 0; k < 8; ++k)
    scp[k] = __builtin_amdgcn_sbfe(static_cast<int>(comp(scv, 2 * (k >> 2) + ((k & 3) >> 1))),
                                   16 * (k & 1) + 8 * p, 8);
#pragma unroll
  for (int k = 0; k < 7; ++k) cf[k] = scp[k] - scp[k + 1];
  cf[7] = scp[7];
  int P[4], is[4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    u32x4 xv[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) xv[g] = *reinterpret_cast<const u32x4*>(xs + 32 * h + 8 * g + 4 * p);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const uint32_t av = comp(a0[h], m), bv = comp(a1[h], m), hv = comp(hb[h], m);
      const uint32_t q0 = (av & 0x0f0f0f0fu) | ((hv << 4) & 0x30303030u);
      const uint32_t q1 = (bv & 0x0f0f0f0fu) | ((hv << 2) & 0x30303030u);
      const uint32_t q2 = ((av >> 4) & 0x0f0f0f0fu) | (hv & 0x30303030u);
      const uint32_t q3 = ((bv >> 4) & 0x0f0f0f0fu) | ((hv >> 2) & 0x30303030u);
      P[m] = pd_dot4(q0, comp(xv[0], m), h == 0 ? 0 : P[m]);
      int v = h == 0 ? __mul24(cf[0], P[m]) : pd_mad24(cf[4], P[m], is[m]);
      P[m] = pd_dot4(q1, comp(xv[1], m), P[m]);
      v = pd_mad24(cf[4 * h + 1], P[m], v);
      P[m] = pd_dot4(q2, comp(xv[2], m), P[m]);
      v = pd_mad24(cf[4 * h + 2], P[m], v);
      P[m] = pd_dot4(q3, comp(xv[3], m), P[m]);
      is[m] = pd_mad24(cf[4 * h + 3], P[m], v);
    }
  }
  const u32x4 b0 = *reinterpret_cast<const u32x4*>(xbs + 8 * p);
  const u32x4 b1 = *reinterpret_cast<const u32x4*>(xbs + 8 * p + 4);
  const int bsv[8] = {static_cast<int>(b0.x), static_cast<int>(b0.y), static_cast<int>(b0.z), static_cast<int>(b0.w),
                      static_cast<int>(b1.x), static_cast<int>(b1.y), static_cast<int>(b1.z), static_cast<int>(b1.w)};
  // lane m = 4p+m' takes sc[2m] and sc[2m+1]: bytes 2(m'&1) and 2(m'&1)+1 of
  // scale dword 2p+(m'>>1)
  const uint32_t slo = p ? scv.z : scv.x, shi = p ? scv.w : scv.y;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int w = static_cast<int>(m < 2 ? slo : shi);
    const int sa = __builtin_amdgcn_sbfe(w, 16 * (m & 1), 8), sb = __builtin_amdgcn_sbfe(w, 16 * (m & 1) + 8, 8);
    is[m] -= 32 * pd_mad24(bsv[2 * m], sa, __mul24(bsv[2 * m + 1], sb));
  }
  *reinterpret_cast<u32x4*>(e + 4 * p) = u32x4{static_cast<uint32_t>(is[0]), static_cast<uint32_t>(is[1]),
                                               static_cast<uint32_t>(is[2]), static_cast<uint32_t>(is[3])};
  if (p == 0) {
    e[8] = __float_as_uint(xd * fp16_to_fp32(static_cast<uint16_t>(dword & 0xffffu)));
    e[9] = 0u;
    e[10] = 0u;
  }
}

// ------------------------------------------------------------ GEMV phase ---
// A phase's rows: up to three sub-regions of its LDS region, each with the
// work group's valid rows, in the order of the phase's row index (chain
// entries and row values).
struct PdPhase {
  const uint8_t* w;        // the region in LDS
  int off0, off1, off2;    // sub-region offsets in the region
  int R0, R1, R2;          // rows allocated (the LDS layout's row stride)
  int ty0, ty1, ty2;       // weight types
  int v0, v1, v2;          // valid rows of each sub-region
  int nsub, nb, rtot;
};

__device__ __forceinline__ PdPhase pd_phase(const uint8_t* w, const PdSub& a, const PdSub& b, const PdSub& c, int v0,
                                            int v1, int v2, int nsub, int nb, int rtot) {
  return PdPhase{w, a.off, b.off, c.off, a.R, b.R, c.R, a.type, b.type, c.type, v0, v1, v2, nsub, nb, rtot};
}

// Integer work of a phase: tasks (sub-region, row, block, half), rows
// fastest so that consecutive lanes read consecutive 16-byte chunks; each
// task's lane sums into its chain entry, (block b, row r) at (b*rtot + r)*12.
// The sub-regions' parameters come from a table in LDS (tab[4i..4i+3]:
// offset, rows allocated, type, valid rows), indexed per task.
__device__ __forceinline__ void pd_tasks(const PdShape& s, const PdPhase& ph, const uint32_t* S, const int* tab,
                                         uint32_t* chain) {
  const int t = static_cast<int>(threadIdx.x);
  // halves of a row-block as tasks of their own when they fit one pass of
  // the work group, else both halves in one task (half the per-task work of
  // finding the row, block and sub-region)
  const int H = (ph.v0 + ph.v1 + ph.v2) * ph.nb * 2 <= 256 ? 2 : 1;
  const int n0 = ph.v0 * ph.nb * H, n1 = ph.nsub > 1 ? ph.v1 * ph.nb * H : 0, n2 = ph.nsub > 2 ? ph.v2 * ph.nb * H : 0;
  // a sub-region of another weight type than the one before starts on a
  // wave boundary, so that no wave runs both types' code
  const int b1 = ph.ty1 != ph.ty0 ? (n0 + 63) & ~63 : n0;
  const int b2 = ph.ty2 != ph.ty1 ? (b1 + n1 + 63) & ~63 : b1 + n1;
  const int nt = b2 + n2;
#pragma unroll 1
  for (int q = t; q < nt; q += 256) {
    const int i = q < b1 ? 0 : q < b2 ? 1 : 2;
    const int qq = q - (i == 0 ? 0 : i == 1 ? b1 : b2);
    if (qq >= (i == 0 ? n0 : i == 1 ? n1 : n2)) continue;  // padding to the wave boundary
    const int off = tab[4 * i], RA = tab[4 * i + 1], ty = tab[4 * i + 2], R = tab[4 * i + 3];
    const int rbase = i == 0 ? 0 : i == 1 ? ph.v0 : ph.v0 + ph.v1;
    const int row = qq % R, bp = qq / R, blk = H == 2 ? bp >> 1 : bp;
    uint32_t* e = chain + (blk * ph.rtot + rbase + row) * 12;
    const float xd = __uint_as_float(S[s.s_xd + blk]);
    auto half = [&](int p) {
      if (ty == MCPM_TYPE_Q4_K)
        q4k_half(ph.w + off, RA, blk, row, p, S + s.s_xs + blk * 68, S + s.s_xbp + blk * 4, xd, e);
      else
        q6k_half(ph.w + off, RA, ph.nb, blk, row, p, S + s.s_xs + blk * 68, S + s.s_xbs + blk * 16, xd, e);
    };
    // both halves of a row-block in one straight run, so that the second's
    // LDS reads can be issued while the first computes
    if (H == 2) {
      half(bp & 1);
    } else {
      half(0);
      half(1);
    }
  }
}

// The float chain over the blocks, in order (the per-token GEMV's TILE
// chain): 4 lanes per row, lane c the accumulators of lane sums c and c+4,
// then ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) by DPP row shifts, plus the
// Q4_K min chain.  Row values to vrow.
__device__ __forceinline__ void pd_chain(const PdPhase& ph, const int* tab, const uint32_t* chain, float* vrow) {
  const int t = static_cast<int>(threadIdx.x), row = t >> 2, c = t & 3;
  if (row >= ph.rtot) return;  // whole groups of 4 lanes
  const int i = row < ph.v0 ? 0 : row < ph.v0 + ph.v1 ? 1 : 2;
  const bool q4 = tab[4 * i + 2] == MCPM_TYPE_Q4_K;
  float a0 = 0.0f, a1 = 0.0f, am = 0.0f;
  const int nb = ph.nb;
#pragma unroll 1
  for (int bq = 0; bq < nb; bq += CHAIN_BATCH_PD) {
    int i0[CHAIN_BATCH_PD], i1[CHAIN_BATCH_PD];
    f32x4 dv[CHAIN_BATCH_PD];
#pragma unroll
    for (int k = 0; k < CHAIN_BATCH_PD; ++k) {
      const uint32_t* e = chain + (min(bq + k, nb - 1) * ph.rtot + row) * 12;
      i0[k] = static_cast<int>(e[c]);
      i1[k] = static_cast<int>(e[c + 4]);
      dv[k] = *reinterpret_cast<const f32x4*>(e + 8);
    }
#pragma unroll
    for (int k = 0; k < CHAIN_BATCH_PD; ++k) {
      if (bq + k < nb) {
        a0 = __builtin_fmaf(dv[k].x, static_cast<float>(i0[k]), a0);
        a1 = __builtin_fmaf(dv[k].x, static_cast<float>(i1[k]), a1);
        am = __builtin_fmaf(-dv[k].y, static_cast<float>(__float_as_int(dv[k].z)), am);
      }
    }
  }
  float v = a0 + a1;
  v = v + dpp_f<0x102>(v);  // row_shl:2
  v = v + dpp_f<0x101>(v);  // row_shl:1
  if (q4) v = v + am;
  if (c == 0) vrow[row] = v;
}

// A Q8_K prologue from fp32 values x[t + 256k] (k < nbx) of every thread:
// RMSNorm with gamma (the 256-slot tree over x[t], x[t+256], ...), then the
// ties-away quantization of each block by a row of 16 lanes (block r16, lane
// j values 16j..16j+15).
__device__ __forceinline__ void pd_norm_quant(const PdShape& s, uint32_t* S, const uint32_t (&xv)[PD_NBX],
                                              const f32x4 (&gam)[4]) {
  const int t = static_cast<int>(threadIdx.x), r16 = t >> 4, j = t & 15;
  float* U = reinterpret_cast<float*>(S + s.s_u);
  float p = 0.0f;
#pragma unroll
  for (int k = 0; k < PD_NBX; ++k) {
    if (k < s.nbx) {
      const float x = __uint_as_float(xv[k]);
      p = p + x * x;
      U[t + 256 * k] = x;
    }
  }
  const float rms = pd_rms(p, s.dim, s.eps, reinterpret_cast<float*>(S + s.s_red));
  if (r16 < s.nbx) {
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 x4 = *reinterpret_cast<const f32x4*>(U + r16 * 256 + 16 * j + 4 * i);
      v[4 * i] = (x4.x * rms) * gam[i].x;
      v[4 * i + 1] = (x4.y * rms) * gam[i].y;
      v[4 * i + 2] = (x4.z * rms) * gam[i].z;
      v[4 * i + 3] = (x4.w * rms) * gam[i].w;
    }
    u32x4 packed;
    float d;
    int gsum;
    quant_block_row16(v, true, packed, d, gsum);
    pd_store_xblock(S, s, r16, j, packed, d, gsum);
  }
  pd_bar();
}

template <bool FS>
__device__ __forceinline__ const uint8_t* pd_slab(const PdArgs& a, int l, int r) {
  const PdShape& s = pd_s<FS>(a);
  return a.slab + (static_cast<size_t>(l) * s.G + blockIdx.x) * s.slab_stride + s.reg_off[r];
}
template <bool FS>
__device__ __forceinline__ void pd_copy_region(const PdArgs& a, uint8_t* LDS, int l, int r) {
  const PdShape& s = pd_s<FS>(a);
  pd_copy(pd_slab<FS>(a, l, r), LDS + s.reg_off[r], r == 2 ? pd_gu(s, static_cast<int>(blockIdx.x)).bytes : s.reg_sz[r]);
}

// Whether chunk owner k (k < the chunk count) stages its layer's chunk
// early, into the gate/up region during the previous layer's D (layer 0's
// at E): where that region holds the attention's staging, on every owner
// but the combining work group (k = W-1), which takes its gate/up copy at
// A and stages into the down region at Q.
__device__ __forceinline__ bool pd_stage_early(const PdShape& s, int k) {
  return s.reg_sz[2] >= PD_ATTN_LDS && k != s.W - 1;
}

// The attention staging of chunk k's owner: the gate/up region when it
// stages early, else the down region.
// Whether the owner of a context's only chunk (k = 0, a first-chunk owner
// with its short gate/up rows) stages at G instead of D, past its gate/up
// rows in that region: its G, with few rows, ends before the others', while
// a copy at D made its D end after theirs.
__device__ __forceinline__ bool pd_solo_stage_g(const PdShape& s, int k, int nch) {
  return nch == 1 && k == 0 && pd_stage_early(s, k) && pd_gu(s, 0).bytes + PD_ATTN_LDS <= s.reg_sz[2];
}

__device__ __forceinline__ int pd_stage_off(const PdShape& s, int k, int nch) {
  return pd_solo_stage_g(s, k, nch) ? s.reg_off[2] + pd_gu(s, 0).bytes
         : pd_stage_early(s, k)     ? s.reg_off[2]
                                    : s.reg_off[3];
}

// Chunk k of layer l's K and V rows of this work group's kv head (context
// pos + 1) into its attention staging.
template <bool FS>
__device__ __forceinline__ void pd_stage_layer(const PdArgs& a, int l, int k, int pos, uint8_t* LDS) {
  const PdShape& s = pd_s<FS>(a);
  const size_t lay = static_cast<size_t>(l) * a.max_seq * s.kvd;
  pd_stage_chunk(a.kc + lay, a.vc + lay, k, pos + 1, s.kvd,
                 static_cast<size_t>(static_cast<int>(blockIdx.x) % PD_XCDS) * s.hd, a.norms,
                 LDS + pd_stage_off(s, k, (pos + ATTN_CHUNK) / ATTN_CHUNK));
}

// Q (kind 0), O (2), G (3) or D (4) of layer l.
template <bool XL, bool FS>
__device__ __forceinline__ bool pd_gemv(const PdArgs& a, int l, int kind, uint8_t* LDS, uint32_t* S, uint32_t tag,
                                        int pos, uint32_t& vit) {
  const PdShape& s = pd_s<FS>(a);
  const PdRows me = pd_rows(s, static_cast<int>(blockIdx.x));
  const int t = static_cast<int>(threadIdx.x), r16 = t >> 4, j = t & 15;
  uint32_t* misc = S + s.s_misc;
  float* vrow = reinterpret_cast<float*>(S + s.s_vrow);
  float* ownx = reinterpret_cast<float*>(S + s.s_ownx);
  float* ownx2 = reinterpret_cast<float*>(S + s.s_ownx2);

  PdPhase ph;
  if (kind == 0) {
    ph = pd_phase(LDS + s.reg_off[0], s.sq, s.sk, s.sv, s.nq, s.nk, s.nk, 3, s.nbx, s.nq + 2 * s.nk);
  } else if (kind == 2) {
    ph = pd_phase(LDS + s.reg_off[1], s.so, s.so, s.so, me.nh, 0, 0, 1, s.nbq, me.nh);
  } else if (kind == 3) {
    const PdGu gu = pd_gu(s, static_cast<int>(blockIdx.x));
    ph = pd_phase(LDS + s.reg_off[2], gu.g, gu.u, gu.u, me.np, me.np, 0, 2, s.nbx, 2 * me.np);
  } else {
    ph = pd_phase(LDS + s.reg_off[3], s.sd, s.sd, s.sd, me.nh, 0, 0, 1, s.nbh, me.nh);
  }

  // the sub-regions' table for the task loop (read after the prologue's
  // barrier)
  int* tab = reinterpret_cast<int*>(misc + 12);
  if (t == 0) {
    tab[0] = ph.off0;
    tab[1] = ph.R0;
    tab[2] = ph.ty0;
    tab[3] = ph.v0;
    tab[4] = ph.off1;
    tab[5] = ph.R1;
    tab[6] = ph.ty1;
    tab[7] = ph.v1;
    tab[8] = ph.off2;
    tab[9] = ph.R2;
    tab[10] = ph.ty2;
    tab[11] = ph.v2;
  }

  // loads that do not depend on the hand-off go first: the RMSNorm gains in
  // the quantization layout, and the RoPE (cos, sin) of the thread's
  // epilogue row
  f32x4 gam[4];
  if (kind == 0 || kind == 3) {
    const float* g = a.norms + (static_cast<size_t>(2 * l) + (kind == 0 ? 0 : 1)) * s.dim;
    if (r16 < s.nbx) {
#pragma unroll
      for (int i = 0; i < 4; ++i) gam[i] = reinterpret_cast<const f32x4*>(g + r16 * 256 + 16 * j)[i];
    }
  }
  float2 cs = make_float2(0.0f, 0.0f);
  if (kind == 0 && t < s.nq + s.nk) {
    const int r = t < s.nq ? me.qr0 + t : me.kr0 + (t - s.nq);
    cs = a.rope[static_cast<size_t>(pos) * (s.hd / 2) + ((r % s.hd) >> 1)];
  }

  // weight copies for later phases, issued while this phase waits for its
  // hand-off (the waves are idle then, and a copy stalls the wave issuing it
  // for most of its transfer): each region after its last use, before the
  // wait of a phase ahead of its next.  Q: this layer's O (and, where the
  // down region is the attention's staging, the chunk's rows); O: the next
  // layer's QKV, this layer's gate/up and down (the attention's staging is
  // done), where every other phase's wait is an all-to-all wait but O's runs
  // beside the attention.  The kv heads' combining work groups (k = W-1)
  // take gate/up at A, while they wait for the chunks' partials, and the
  // rest at G; the owner of a context's only chunk, which reaches O last,
  // takes gate/up (its own rows only) at O and the rest, with its next
  // chunk's staging, at G, where its few FFN rows leave it time.  D: the
  // other chunk owners' next attention rows, into the gate/up region.
  if (kind == 0) {
    pd_copy_region<FS>(a, LDS, l, 1);
    // this layer's attention chunk (the down region is free until G), where
    // it was not staged at the previous layer's D
    if (me.k < (pos + ATTN_CHUNK) / ATTN_CHUNK && !pd_stage_early(s, me.k)) pd_stage_layer<FS>(a, l, me.k, pos, LDS);
  }
  // the next layer's attention chunk, into the gate/up region (free from the
  // end of G until this work group's next gate/up copy at O, after A), so
  // that the copy lands during this phase's wait instead of the next Q's
  if (kind == 4 && l + 1 < a.s.L && me.k < (pos + ATTN_CHUNK) / ATTN_CHUNK && pd_stage_early(s, me.k) &&
      !pd_solo_stage_g(s, me.k, (pos + ATTN_CHUNK) / ATTN_CHUNK))
    pd_stage_layer<FS>(a, l + 1, me.k, pos, LDS);
  // (with one chunk the combining work group has nothing to wait for at A,
  // where the chunk's owner finishes the head, and takes its copies here)
  const bool solo = pos < ATTN_CHUNK && me.k == 0;
  // (with one chunk, the plain work groups' next QKV at D: O's wait ends
  // with its copies, the attention being short)
  if (kind == 2 && (me.k != s.W - 1 || pos < ATTN_CHUNK)) {
    if (l + 1 < a.s.L && !solo && pos >= ATTN_CHUNK) pd_copy_region<FS>(a, LDS, l + 1, 0);
    pd_copy_region<FS>(a, LDS, l, 2);
    if (!solo) pd_copy_region<FS>(a, LDS, l, 3);
  }
  if (kind == 4 && l + 1 < a.s.L && pos < ATTN_CHUNK && !solo) pd_copy_region<FS>(a, LDS, l + 1, 0);
  // the combining work group's next QKV and down copies (at A they would
  // lengthen its wait for the partials; where it owns a chunk its staging is
  // the down region until then), and those of the single chunk's owner
  if (kind == 3 && ((me.k == s.W - 1 && pos >= ATTN_CHUNK) || solo)) {
    if (l + 1 < a.s.L) pd_copy_region<FS>(a, LDS, l + 1, 0);
    pd_copy_region<FS>(a, LDS, l, 3);
  }
  if (kind == 3 && l + 1 < a.s.L && pd_solo_stage_g(s, me.k, (pos + ATTN_CHUNK) / ATTN_CHUNK))
    pd_stage_layer<FS>(a, l + 1, me.k, pos, LDS);

  // hand-off and prologue: the Q8_K activations into the scratch
  if (kind == 0 || kind == 3) {
    uint32_t xv[PD_NBX];
    const int nbx = s.nbx;
    if (!pd_poll<PD_NBX>(a, kind == 0 ? a.rx : a.rx2, tag, [&](int k) { return k < nbx ? t + 256 * k : -1; }, xv,
                         misc, vit))
      return false;
    pd_norm_quant(s, S, xv, gam);
  } else if (kind == 2) {
    uint32_t v[3];
    const int n = s.nbq * PD_REC_BLK;
    if (!pd_poll<3>(a, a.ratt, tag, [&](int k) { return t + 256 * k < n ? t + 256 * k : -1; }, v, misc, vit))
      return false;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const int i = t + 256 * k;
      if (i < n) {
        const int blk = i / PD_REC_BLK, w = i - blk * PD_REC_BLK;
        if (w == 0) S[s.s_xd + blk] = v[k];
        else if (w <= 64) S[s.s_xs + blk * 68 + w - 1] = v[k];
        else if (w <= 80) S[s.s_xbs + blk * 16 + w - 65] = v[k];
        else S[s.s_xbp + blk * 4 + w - 81] = v[k];
      }
    }
    pd_bar();
  } else {
    // h in rounds of up to 16 blocks: records t + 256k of the round (lanes
    // on consecutive records) into the staging area, then block r16 of the
    // round quantized by its row of 16 lanes (zero past ffn).  Up to 24
    // blocks every record is waited for at once, so the second round costs
    // no second round trip, and where the O weights' region holds the blocks
    // past the 16th the two rounds are one.
    const int nbh = s.nbh, ffn = s.ffn;
    float* U = reinterpret_cast<float*>(S + s.s_u);
    auto quant_round = [&](int b0, int nbr) {
      pd_bar();
      if (r16 < nbr) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x4 x4 = *reinterpret_cast<const f32x4*>(U + r16 * 256 + 16 * j + 4 * i);
          v[4 * i] = x4.x;
          v[4 * i + 1] = x4.y;
          v[4 * i + 2] = x4.z;
          v[4 * i + 3] = x4.w;
        }
        u32x4 packed;
        float d;
        int gsum;
        quant_block_row16(v, true, packed, d, gsum);
        pd_store_xblock(S, s, b0 + r16, j, packed, d, gsum);
      }
      pd_bar();  // the staging area's readers are done before the next round
    };
    if (nbh <= 24) {
      uint32_t hv[24];
      if (!pd_poll<24>(a, a.rh, tag,
                       [&](int k) {
                         const int e = t + 256 * k;
                         return k < nbh && e < ffn ? e : -1;
                       },
                       hv, misc, vit))
        return false;
      if (nbh > 16 && (nbh - 16) * QK_K * 4 <= s.reg_sz[1]) {
        // one round: blocks 16.. staged in the O weights' region (read at O,
        // next written by the next layer's Q copy), the rows of waves 0 and 1
        // quantizing two blocks each in one straight run
        float* U2 = reinterpret_cast<float*>(LDS + s.reg_off[1]);
#pragma unroll
        for (int k = 0; k < 16; ++k) U[t + 256 * k] = __uint_as_float(hv[k]);
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (k < nbh - 16) U2[t + 256 * k] = __uint_as_float(hv[16 + k]);
        pd_bar();
        auto ld16 = [&](const float* src, float (&v)[16]) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const f32x4 x4 = *reinterpret_cast<const f32x4*>(src + 16 * j + 4 * i);
            v[4 * i] = x4.x;
            v[4 * i + 1] = x4.y;
            v[4 * i + 2] = x4.z;
            v[4 * i + 3] = x4.w;
          }
        };
        float v0[16];
        ld16(U + r16 * 256, v0);
        u32x4 p0;
        float d0;
        int g0;
        if (r16 < 8) {  // waves 0 and 1; rows past the last block quantize a copy of it and store nothing
          float v1[16];
          ld16(U2 + min(r16, nbh - 17) * 256, v1);
          u32x4 p1;
          float d1;
          int g1;
          quant_block_row16(v0, true, p0, d0, g0);
          quant_block_row16(v1, true, p1, d1, g1);
          pd_store_xblock(S, s, r16, j, p0, d0, g0);
          if (r16 < nbh - 16) pd_store_xblock(S, s, 16 + r16, j, p1, d1, g1);
        } else {
          quant_block_row16(v0, true, p0, d0, g0);
          pd_store_xblock(S, s, r16, j, p0, d0, g0);
        }
        pd_bar();
      } else {
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          const int b0 = 16 * rr, nbr = min(16, nbh - b0);
          if (nbr > 0) {  // uniform
#pragma unroll
            for (int k = 0; k < 16; ++k)
              if (k < nbr) U[t + 256 * k] = __uint_as_float(hv[b0 + k < 24 ? b0 + k : 0]);
            quant_round(b0, nbr);
          }
        }
      }
    } else {
#pragma unroll 1
      for (int b0 = 0; b0 < nbh; b0 += 16) {
        const int nbr = min(16, nbh - b0), e0 = b0 * 256;
        uint32_t hv[16];
        if (!pd_poll<16>(a, a.rh, tag,
                         [&](int k) {
                           const int e = e0 + t + 256 * k;
                           return k < nbr && e < ffn ? e : -1;
                         },
                         hv, misc, vit))
          return false;
#pragma unroll
        for (int k = 0; k < 16; ++k)
          if (k < nbr) U[t + 256 * k] = __uint_as_float(hv[k]);
        quant_round(b0, nbr);
      }
    }
  }

  uint32_t* chain = S + s.s_u;  // the prologue's x staging is no longer read
  pd_tasks(s, ph, S, tab, chain);
  pd_bar();
  pd_chain(ph, tab, chain, vrow);
  pd_bar();

  // epilogues
  if (kind == 0) {
    if (t < ph.rtot) {
      const float v = vrow[t];
      const int kvd = s.kvd;
      const size_t row_off = static_cast<size_t>(l) * a.max_seq * kvd + static_cast<size_t>(pos) * kvd;
      uint64_t* qrec = a.rqkv + static_cast<size_t>(me.kvh) * (s.gh + 2 * s.hd);
      if (t < s.nq + s.nk) {
        // adjacent-pair RoPE (src/ops/ops.cpp:502-516) on q and k rows
        const float partner = vrow[t ^ 1];
        const int r = t < s.nq ? me.qr0 + t : me.kr0 + (t - s.nq);
        const int i = r % s.hd;
        float o;
        if ((i & 1) == 0) o = v * cs.x - partner * cs.y;
        else o = partner * cs.y + v * cs.x;
        if (t < s.nq) {
          rec_stf_xcd<XL>(qrec + (r - me.kvh * s.gh), o, tag);
        } else {
          a.kc[row_off + r] = o;
          rec_stf_xcd<XL>(qrec + s.gh + (r - me.kvh * s.hd), o, tag);
        }
      } else {
        const int r = me.kr0 + (t - s.nq - s.nk);
        a.vc[row_off + r] = v;
        rec_stf_xcd<XL>(qrec + s.gh + s.hd + (r - me.kvh * s.hd), v, tag);
      }
    }
  } else if (kind == 2) {
    if (t < me.nh) {
      const float x2 = ownx[t] + vrow[t];
      ownx2[t] = x2;
      rec_stf(a.rx2 + me.hr0 + t, x2, tag);
    }
  } else if (kind == 3) {
    if (t < me.np) {
      const float g = vrow[t], u = vrow[me.np + t];
      const float silu = g / (1.0f + exp_f32(-g));
      rec_stf(a.rh + me.fp0 + t, silu * u, tag);
    }
  } else {
    if (t < me.nh) {
      const float x = ownx2[t] + vrow[t];
      ownx[t] = x;
      if (l + 1 < a.s.L) rec_stf(a.rx + me.hr0 + t, x, tag + 1);
      else a.x_out[me.hr0 + t] = x;
    }
  }
  return true;
}

// Register slots of K and V rows at position T-1 (and the clamped slots past
// it) from the rows handed over by the QKV phase (LDS kr, vr).
__device__ __forceinline__ void pd_fill_last(AttnRegs<4>& R, const float* kr, const float* vr, int c, int T) {
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int f = static_cast<int>(threadIdx.x) + 256 * u;
    const int jr = f >> 4, c4 = f & 15;
    if (min(c * ATTN_CHUNK + jr, T - 1) == T - 1) {
      R.k[u] = *reinterpret_cast<const f32x4*>(kr + 4 * c4);
      R.v[u] = *reinterpret_cast<const f32x4*>(vr + 4 * c4);
    }
  }
}

// The attention of layer l (src/ops/ops.cpp:537-628) for kv head h = b % 8,
// head_dim 64, a head group of 256 outputs (gh).  Chunk c of 64 positions on
// work group (h, c mod W); work group (h, W-1) combines the head's chunks.
// Below W chunks the combining work group has no chunk of its own and would
// wait idle for the partials, so it takes its gate/up copy here (its next
// QKV and down copies at G: at A they would end its wait later than the
// partials, competing with every other work group's copies at O).  With
// one chunk the chunk's owner finishes the head and no work group combines.
template <bool XL, bool FS>
__device__ __forceinline__ bool pd_attention(const PdArgs& a, int l, uint8_t* LDS, uint32_t* S, uint32_t tag, int T,
                                             uint32_t& vit) {
  const PdShape& s = pd_s<FS>(a);
  const int t = static_cast<int>(threadIdx.x), h = static_cast<int>(blockIdx.x) % PD_XCDS,
            k = static_cast<int>(blockIdx.x) / PD_XCDS, W = s.W;
  uint32_t* misc = S + s.s_misc;
  const int nch = (T + ATTN_CHUNK - 1) / ATTN_CHUNK;
  // one chunk: its owner finishes the head (the combine of one chunk is the
  // chunk's own o_c / z_c), so no partials go to the combining work group
  const bool combiner = k == W - 1 && nch > 1;
  if (k >= nch && !combiner) return true;  // no chunk of this context
  if (combiner) pd_copy_region<FS>(a, LDS, l, 2);  // (its next QKV and down weights at G)
  constexpr int HD = 64, GH = 256, OPT = ATTN_MAX_GROUP * HD / 256;
  const int group = s.group, kvd = s.kvd;
  const AttnLds<HD> A(reinterpret_cast<float*>(LDS + pd_stage_off(s, k, nch)));
  float* kr = reinterpret_cast<float*>(S + s.s_u);
  float* vr = kr + HD;
  float* sX = vr + HD;       // [GH] the combined output
  float* sO = sX + GH;       // [2][GH] this work group's chunks' o_c
  float* sM = sO + 2 * GH;   // [max_chunks][group] m_c (combining work group)
  float* sZ = sM + 64 * ATTN_MAX_GROUP;
  if (k < nch) {
    const size_t lay = static_cast<size_t>(l) * a.max_seq * kvd;
    const float* kc = a.kc + lay;
    const float* vc = a.vc + lay;
    AttnRegs<4> R;
    const size_t head_off = static_cast<size_t>(h) * HD;
    // chunk k's rows before pos are in LDS since the QKV phase (pd_stage_chunk);
    // q of the head group and the K and V rows at pos, from the QKV phase
    constexpr int NREC = GH + 2 * HD;
    uint32_t qv[2];
    if (!pd_poll<2>(a, a.rqkv + static_cast<size_t>(h) * NREC, tag,
                    [&](int kk) { return t + 256 * kk < NREC ? t + 256 * kk : -1; }, qv, misc, vit))
      return false;
    A.sQ[(t / HD) * HD + t % HD] = __uint_as_float(qv[0]);
    if (t < 2 * HD) kr[t] = __uint_as_float(qv[1]);  // kr, vr contiguous
    pd_bar();
    const float scale = 1.0f / sqrtf(static_cast<float>(HD));
#pragma unroll 1
    for (int cc = 0; cc < 2; ++cc) {
      const int c = k + W * cc;
      if (c >= nch) break;  // uniform
      if (cc == 0) {
        // row T-1 of the staged chunk from the hand-off
        if (c == nch - 1 && t < 2 * HD) {
          const int jr = T - 1 - c * ATTN_CHUNK;
          if (t < HD) A.sK[jr * (HD + 4) + t] = kr[t];
          else A.sV[jr * HD + (t - HD)] = vr[t - HD];
        }
      } else {
        if (c == nch - 1) pd_fill_last(R, kr, vr, c, T);
        pd_bar();  // readers of the previous chunk are done
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int f = t + 256 * u, jr = f >> 4, c4 = f & 15;
          *reinterpret_cast<f32x4*>(&A.sK[jr * (HD + 4) + c4 * 4]) = R.k[u];
          *reinterpret_cast<f32x4*>(&A.sV[jr * HD + c4 * 4]) = R.v[u];
        }
      }
      if (c + W < nch) attn_load_chunk<4, true>(R, kc, vc, c + W, T, kvd, head_off, HD / 4, ATTN_CHUNK * HD / 4);
      pd_bar();
      float o[OPT];
      attn_token_chunk<HD, OPT, true>(A.sK, A.sV, A.sQ, A.sE, A.sMZ + cc * ATTN_MAX_GROUP, c, T, group, HD, GH,
                                      scale, o, t);
      sO[cc * GH + t] = o[0];
    }
    pd_bar();  // (m_c, z_c) of every head, every chunk's o_c
  }
  // the head group's Q8_K block (ties even) of sX on lanes 0..15, to its
  // attention-output records
  auto publish = [&]() {
    if (t < 16) {
      const int j = t;
      float v[16];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 x4 = *reinterpret_cast<const f32x4*>(sX + 16 * j + 4 * i);
        v[4 * i] = x4.x;
        v[4 * i + 1] = x4.y;
        v[4 * i + 2] = x4.z;
        v[4 * i + 3] = x4.w;
      }
      u32x4 packed;
      float d;
      int gsum;
      quant_block_row16(v, false, packed, d, gsum);
      const int vs = gsum + dpp_i<DPP_XOR1>(gsum);
      const uint32_t w = (static_cast<uint32_t>(vs) & 0xffffu) | (static_cast<uint32_t>(dpp_i<DPP_XOR2>(vs)) << 16);
      uint64_t* rb = a.ratt + static_cast<size_t>(h) * PD_REC_BLK;
      rec_st(rb + 1 + 4 * j, packed.x, tag);
      rec_st(rb + 2 + 4 * j, packed.y, tag);
      rec_st(rb + 3 + 4 * j, packed.z, tag);
      rec_st(rb + 4 + 4 * j, packed.w, tag);
      rec_st(rb + 65 + j, static_cast<uint32_t>(gsum), tag);
      if (j == 0) rec_stf(rb, d, tag);
      if ((j & 3) == 0) rec_st(rb + 81 + (j >> 2), w, tag);
    }
  };
  if (nch == 1) {
    // the combining work group's arithmetic on one chunk: m = m_0,
    // f = exp(m_0 - m), Z = fma(z_0, f, 0), O = fma(o_0, f, 0), out = O / Z
    const float2 mz = A.sMZ[t / HD];
    const float f = exp_f32(mz.x - mz.x);
    sX[t] = __builtin_fmaf(sO[t], f, 0.0f) / __builtin_fmaf(mz.y, f, 0.0f);
    pd_bar();
    publish();
    // the staging (read above) is overwritten by the next phase's copies
    pd_bar();
    return true;
  }
  const int ppc = s.part_stride;  // o_c (GH), m_c (group), z_c (group), in whole lines
  uint64_t* part = a.rpart + static_cast<size_t>(h) * a.s.max_chunks * ppc;
  if (!combiner) {
#pragma unroll 1
    for (int cc = 0; cc < 2; ++cc) {
      const int c = k + W * cc;
      if (c >= nch) break;
      uint64_t* pr = part + static_cast<size_t>(c) * ppc;
      rec_stf_xcd<XL>(pr + t, sO[cc * GH + t], tag);
      if (t < group) {
        const float2 mz = A.sMZ[cc * ATTN_MAX_GROUP + t];
        rec_stf_xcd<XL>(pr + GH + t, mz.x, tag);
        rec_stf_xcd<XL>(pr + GH + group + t, mz.y, tag);
      }
    }
    // (m_c, z_c) are read from the staging, which the next phase's weight
    // copies overwrite
    pd_bar();
    return true;
  }
  // The combining work group takes the chunks in chunk order with the
  // per-token path's arithmetic: m = max m_c; f_c = exp(m_c - m);
  // Z = fma(z_c, f_c, Z); O = fma(o_c, f_c, O); out = O / Z.  Its own chunks
  // (W-1 and 2W-1, where they exist) come from LDS, the others from their
  // records: in one wait, every chunk's (m_c, z_c) (one (chunk, head) per
  // thread, into LDS) and this thread's o_c of the first 8 chunks; later
  // chunks' o_c in batches of 8.  m and the f_c are formed once per head,
  // on its wave (lane c: chunk c; the max is exact in any order), so each
  // step of the chains is two fmas.
  constexpr int B = 8;
  const int own0 = W - 1, own1 = 2 * W - 1;
  bool ok = true;
  const int hh = t / HD;
  uint32_t rv[2 + B];
  {
    const int cq = t / group, hq = t - cq * group;
    const bool mine = cq == own0 || cq == own1;
    const bool mz_rec = t < nch * group && !mine;
    const uint64_t* p[2 + B];
    p[0] = part + static_cast<size_t>(min(cq, nch - 1)) * ppc + GH + hq;
    p[1] = p[0] + group;
    uint32_t mask = mz_rec ? 3u : 0u;
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int c = i;
      p[2 + i] = part + static_cast<size_t>(min(c, nch - 1)) * ppc + t;
      if (c < nch && c != own0 && c != own1) mask |= 1u << (2 + i);
    }
    ok = pd_wait_m<2 + B>(p, mask, tag, a.spin_limit, rv);
    if (t < nch * group) {
      float mc, zc;
      if (mine) {
        const float2 mz = A.sMZ[(cq == own0 ? 0 : ATTN_MAX_GROUP) + hq];
        mc = mz.x;
        zc = mz.y;
      } else {
        mc = __uint_as_float(rv[0]);
        zc = __uint_as_float(rv[1]);
      }
      sM[t] = mc;
      sZ[t] = zc;
    }
  }
  if (pd_any(!ok, misc + 4, vit)) {
    if (t == 0) st_u32c(a.err, 1u);
    return false;
  }
  {
    // head hh's f_c in place of its m_c (read and written by its own wave;
    // nch <= 64)
    const int c = t & 63;
    const float mc = c < nch ? sM[c * group + hh] : -__builtin_inff();
    const float m = wave_max_fast(mc);
    if (c < nch) sM[c * group + hh] = exp_f32(mc - m);
    wave_sync();
  }
  float Z = 0.0f, O = 0.0f;
  auto step = [&](int c, float o) {
    const float f = sM[c * group + hh];
    Z = __builtin_fmaf(sZ[c * group + hh], f, Z);
    O = __builtin_fmaf(o, f, O);
  };
#pragma unroll
  for (int i = 0; i < B; ++i) {
    const int c = i;
    if (c < nch) step(c, c == own0 ? sO[t] : c == own1 ? sO[GH + t] : __uint_as_float(rv[2 + i]));
  }
#pragma unroll 1
  for (int c0 = B; c0 < nch && ok; c0 += B) {
    const uint64_t* pb[B];
    uint32_t mask = 0;
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int c = c0 + i;
      pb[i] = part + static_cast<size_t>(min(c, nch - 1)) * ppc + t;
      if (c < nch && c != own0 && c != own1) mask |= 1u << i;
    }
    uint32_t ov[B];
    ok = pd_wait_m<B>(pb, mask, tag, a.spin_limit, ov);
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int c = c0 + i;
      if (ok && c < nch) step(c, c == own0 ? sO[t] : c == own1 ? sO[GH + t] : __uint_as_float(ov[i]));
    }
  }
  sX[t] = O / Z;
  if (pd_any(!ok, misc + 4, vit)) {  // (its barrier also orders sX)
    if (t == 0) st_u32c(a.err, 1u);
    return false;
  }
  publish();
  return true;
}

// One launch per token: every layer, from the embedding to the last layer's
// x (x_out).
template <bool XL, bool FS>
__global__ void __launch_bounds__(256) k_decode_persist(const PdArgs a) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t LDS[];
  uint32_t* S = reinterpret_cast<uint32_t*>(LDS + pd_s<FS>(a).scr_off);
  uint32_t* misc = S + pd_s<FS>(a).s_misc;
  const int t = static_cast<int>(threadIdx.x);
  if (t == 0) {
    misc[0] = 0u;
    misc[1] = ld_u32c(a.epoch);
    // the XCD (XCC_ID register, bits 3:0) must be the one seen at set-up,
    // where this work group's XCD-local records are read
    if (XL && static_cast<int>(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15u) != a.xcc[blockIdx.x]) {
      misc[0] = 1u;
      st_u32c(a.err, 2u);
    }
  }
  pd_bar();
  if (misc[0]) return;
  const uint32_t ep = misc[1];
  const int pos = a.state[1], T = pos + 1, L = a.s.L;
  const uint32_t tag0 = ep * static_cast<uint32_t>(L + 1) + 1u;
  uint32_t vit = 0;
  // E: this work group's embedding values, then layer 0's QKV and O weights
  {
    const PdRows me = pd_rows(pd_s<FS>(a), static_cast<int>(blockIdx.x));
    float* ownx = reinterpret_cast<float*>(S + pd_s<FS>(a).s_ownx);
    if (t < me.nh) {
      const int r = me.hr0 + t;
      const float x = dequant_value(a.embd, a.state[0], r / QK_K, r % QK_K);
      ownx[t] = x;
      rec_stf(a.rx + r, x, tag0);
    }
  }
  pd_copy_region<FS>(a, LDS, 0, 0);
  {
    const int k = static_cast<int>(blockIdx.x) / PD_XCDS;
    if (k < (pos + ATTN_CHUNK) / ATTN_CHUNK && pd_stage_early(pd_s<FS>(a), k)) pd_stage_layer<FS>(a, 0, k, pos, LDS);
  }
  // one loop over the phases, so that each phase's code exists once
#pragma unroll 1
  for (int ph = 0; ph < 5 * L; ++ph) {
    const int l = ph / 5, kind = ph - 5 * l;
    const uint32_t tag = tag0 + static_cast<uint32_t>(l);
    const bool ok =
        kind == 1 ? pd_attention<XL, FS>(a, l, LDS, S, tag, T, vit) : pd_gemv<XL, FS>(a, l, kind, LDS, S, tag, pos, vit);
    if (!ok) return;
  }
  // every work group read the launch count before its first hand-off, and
  // this work group's last wait needed every work group's output of the
  // phase before, so none reads the count any more
  if (blockIdx.x == 0 && t == 0) st_u32c(a.epoch, ep + 1u);
}

// Slab chunk i (16 bytes) of work group blockIdx.y in layer blockIdx.z.
__global__ void k_build_slab(const PdShape s, const PdLayer* __restrict__ layers, uint8_t* __restrict__ slab) {
  const int b = static_cast<int>(blockIdx.y), l = static_cast<int>(blockIdx.z);
  const int i = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  if (i * 16 >= s.slab_stride) return;
  const PdLayer& Ly = layers[l];
  const WView* wv[7] = {&Ly.q, &Ly.k, &Ly.v, &Ly.o, &Ly.g, &Ly.u, &Ly.d};
  const int rows[7] = {Ly.q.rows, Ly.k.rows, Ly.v.rows, Ly.o.rows, Ly.g.rows, Ly.u.rows, Ly.d.rows};
  const PdSrc src = pd_slab_src(s, b, i * 16, rows);
  u32x4 out = u32x4{0u, 0u, 0u, 0u};
  if (src.tensor >= 0) {
    const WView& w = *wv[src.tensor];
    const uint8_t* plane = src.plane == 0 ? w.p0 : src.plane == 1 ? w.p1 : src.plane == 2 ? w.p2 : w.p3;
    if (src.n == 1) {
      out = *reinterpret_cast<const u32x4*>(plane + src.src[0]);
    } else {
      uint32_t dv[4];
      for (int k = 0; k < 4; ++k)
        dv[k] = src.src[k] < 0 ? 0u
                               : static_cast<uint32_t>(plane[src.src[k]]) | (static_cast<uint32_t>(plane[src.src[k] + 1]) << 8);
      out = u32x4{dv[0], dv[1], dv[2], dv[3]};
    }
  }
  *reinterpret_cast<u32x4*>(slab + (static_cast<size_t>(l) * s.G + b) * s.slab_stride + static_cast<size_t>(i) * 16) = out;
}

}  // namespace

// ------------------------------------------------------------------ host ---

namespace {
// Record counts of the arrays rx, rx2, rh, rqkv, rpart, ratt, each rounded
// to whole cache lines, so that the blocks stored at workgroup scope (a kv
// head's q/k/v rows, a chunk's partials) share no line with another XCD's.
void pd_record_arrays(const PdShape& s, size_t (&n)[6]) {
  const size_t v[6] = {static_cast<size_t>(s.dim), static_cast<size_t>(s.dim), static_cast<size_t>(s.ffn),
                       static_cast<size_t>(s.nkv) * (s.gh + 2 * s.hd),
                       static_cast<size_t>(s.nkv) * s.max_chunks * s.part_stride,
                       static_cast<size_t>(s.nbq) * PD_REC_BLK};
  for (int i = 0; i < 6; ++i) n[i] = (v[i] + PD_REC_LINE - 1) / PD_REC_LINE * PD_REC_LINE;
}

__global__ void k_xcd_probe(int* xcc) {
  if (threadIdx.x == 0) xcc[blockIdx.x] = static_cast<int>(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15u);
}
}  // namespace

size_t pd_records(const PdShape& s) {
  size_t n[6], tot = 0;
  pd_record_arrays(s, n);
  for (size_t v : n) tot += v;
  return tot;
}

void pd_bind_records(PdArgs& a, uint64_t* base) {
  size_t n[6];
  pd_record_arrays(a.s, n);
  uint64_t** arr[6] = {&a.rx, &a.rx2, &a.rh, &a.rqkv, &a.rpart, &a.ratt};
  for (int i = 0; i < 6; ++i) {
    *arr[i] = base;
    base += n[i];
  }
}

hipError_t pd_probe_xcd(int G, int* xcc, hipStream_t st, bool& same) {
  same = false;
  hipLaunchKernelGGL(k_xcd_probe, dim3(G), dim3(256), 0, st, xcc);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  std::vector<int> h(G);
  e = hipMemcpyAsync(h.data(), xcc, G * sizeof(int), hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) return e;
  same = true;
  for (int b = 0; b < G; ++b) same = same && h[b] == h[b % PD_XCDS];
  return hipSuccess;
}

hipError_t launch_build_slab(const PdShape& s, const PdLayer* d_layers, uint8_t* slab, hipStream_t st) {
  const int chunks = s.slab_stride / 16;
  hipLaunchKernelGGL(k_build_slab, dim3((chunks + 255) / 256, s.G, s.L), dim3(256), 0, st, s, d_layers, slab);
  return hipGetLastError();
}

hipError_t prepare_decode_persist(const PdShape& s) {
  for (const void* k : {reinterpret_cast<const void*>(k_decode_persist<false, false>),
                        reinterpret_cast<const void*>(k_decode_persist<true, false>),
                        reinterpret_cast<const void*>(k_decode_persist<false, true>),
                        reinterpret_cast<const void*>(k_decode_persist<true, true>)}) {
    const hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, s.lds_bytes);
    if (e != hipSuccess) return e;
    // every work group must be resident at once: at least one per CU
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k, 256, s.lds_bytes) != hipSuccess || occ < 1)
      return hipErrorNotSupported;
  }
  return hipSuccess;
}

hipError_t launch_decode_persist(const PdArgs& a, hipStream_t st) {
  // the instance compiled for the fixed plan where the launch's plan is it
  const dim3 g(a.s.G), b(256);
  const size_t lds = static_cast<size_t>(a.s.lds_bytes);
  if (pd_fixed_shape(a.s)) {
    if (a.xcd_local) launch_kernel(k_decode_persist<true, true>, g, b, lds, st, a);
    else launch_kernel(k_decode_persist<false, true>, g, b, lds, st, a);
  } else {
    if (a.xcd_local) launch_kernel(k_decode_persist<true, false>, g, b, lds, st, a);
    else launch_kernel(k_decode_persist<false, false>, g, b, lds, st, a);
  }
  return hipGetLastError();
}

}  // namespace mcpm
