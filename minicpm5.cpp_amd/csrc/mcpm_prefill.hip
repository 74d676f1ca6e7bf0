// mcpm_prefill.hip -- batched prompt processing (prefill) for gfx950.
//
// The reference prefills by calling forward() once per prompt token
// (src/chat_session.cpp:154-160).  Here the prompt's tokens go through each
// layer together, and every number that reaches the KV cache is the one the
// per-token decode path produces:
//  * activations are quantized per token exactly as the GEMV prologues do
//    (same RMS tree, same Q8_K rounding), into fp16 copies of the int8 codes;
//  * a row dot keeps the reference's AVX2 structure: per 256-block the eight
//    integer lane sums isum[m] (lane m: bytes 4m..4m+3 of every 32-byte
//    group), then acc[m] = fma(d_x*d_w, float(isum[m]), acc[m]) over blocks in
//    order, Q4_K's min chain, and ((a0+a4)+(a2+a6))+((a1+a5)+(a3+a7));
//  * isum[m] for 16 rows x 16 tokens is one v_mfma_f32_16x16x32_f16: K runs
//    over lane m's 32 bytes (8 sub-blocks x 4) with A = sub-block scale x
//    weight code and B = activation code.  Every product is an integer of at
//    most 2048 in magnitude (exact in fp16) and every sum stays below 2^24
//    (exact in fp32), so the MFMA result is isum[m] itself.  Q4_K: sc*q <= 945.
//    Q6_K: the reference sums sc*q*x over lane m's bytes (q in 0..63) and
//    subtracts 32*(sc[2m]*bsums[2m] + sc[2m+1]*bsums[2m+1]) -- sub-block m's
//    offset, added into lane m -- then converts the int32 sum to float.
//    Written as S + 16*T with q = ql + 16*qh (ql the low 4 bits, qh the high
//    2): S = sum over lane m of sc*ql*x (|sc*ql| <= 1920, |S| < 2^23), T =
//    sum over lane m of sc*qh*x - 2*C (|sc*qh| <= 384), C = sub-block m's
//    sc*bsums pair, fed in as T's accumulator from one more MFMA (|T| <
//    2^22).  Three MFMAs, all exact; fma(16, T, S) rounds S + 16*T once, to
//    nearest even, as the reference's int32 -> float conversion of the same
//    integer does.
//  * Q4_K's min sum (sum over sub-blocks of mn * pair-sum of bsums) is one
//    more MFMA: A = mn[k/2] for k < 16, B = bsums[k].
// Attention per token is the decode kernel at that token's position.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <type_traits>

#include "mcpm_device.h"

namespace mcpm {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

// ------------------------------------------------------------- embedding ---
// Row tokens[t] of the embedding, dequantized into x[t] (grid: blocks x tokens).
__global__ void __launch_bounds__(256) k_embed_batch(const WView w, const int* __restrict__ tokens, int dim,
                                                     float* __restrict__ x) {
  const int t = blockIdx.y;
  const int i = blockIdx.x * QK_K + threadIdx.x;
  if (i < dim) x[static_cast<size_t>(t) * dim + i] = dequant_value(w, tokens[t], blockIdx.x, threadIdx.x);
}

// ------------------------------------------------------------- quantize ----
// Per token (one work group each): the Q8_K quantization of the GEMV
// prologues, written as fp16 codes [t][K], d [t][nb] and fp16 bsums
// [t][nb][16].  mode: PRO_QUANT_EVEN / PRO_QUANT_AWAY / PRO_NORM_AWAY /
// PRO_NORM_EVEN, or QB_SWIGLU: v = silu(g)*u (decode's gate/up epilogue) for
// i < n_valid and 0 beyond, then ties-away (decode's down prologue).
constexpr int QB_SWIGLU = 100;

__global__ void __launch_bounds__(256) k_quant_batch(const float* __restrict__ x, const float* __restrict__ u,
                                                     int ld_x, const float* __restrict__ gamma, float eps, int dim,
                                                     int n_valid, int mode, _Float16* __restrict__ xh,
                                                     float* __restrict__ xd, _Float16* __restrict__ xbs) {
  __shared__ float red[260];
  const int t = blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const float* xt = x + static_cast<size_t>(t) * ld_x;
  const float* ut = u ? u + static_cast<size_t>(t) * ld_x : nullptr;
  const bool norm = (mode == PRO_NORM_AWAY || mode == PRO_NORM_EVEN);
  const bool away = (mode == PRO_QUANT_AWAY || mode == PRO_NORM_AWAY || mode == QB_SWIGLU);
  float rms = 1.0f;
  if (norm) rms = block_rms_scale(xt, dim, eps, red);
  const int nb = dim / QK_K;
  for (int b = wave; b < nb; b += 4) {
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = b * QK_K + 4 * lane + k;
      if (mode == QB_SWIGLU) {
        float h = 0.0f;
        if (i < n_valid) {
          const float g = xt[i];
          const float silu = g / (1.0f + exp_f32(-g));
          h = silu * ut[i];
        }
        v[k] = h;
      } else {
        v[k] = i < n_valid ? xt[i] : 0.0f;
        if (norm) v[k] = (v[k] * rms) * gamma[i];
      }
    }
    uint32_t packed;
    float d;
    int gsum;
    quant_block_wave(v, away, packed, d, gsum);
    _Float16* o = xh + static_cast<size_t>(t) * dim + b * QK_K + 4 * lane;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      o[k] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>((packed >> (8 * k)) & 0xffu)));
    if ((lane & 3) == 0) xbs[(static_cast<size_t>(t) * nb + b) * 16 + (lane >> 2)] = static_cast<_Float16>(gsum);
    if (lane == 0) xd[static_cast<size_t>(t) * nb + b] = d;
  }
}

// k_quant_batch for up to 4*MAXB blocks per token, with every global load
// issued at the start: wave w holds blocks w, w+4, ... (lane l: values 4l ..
// 4l+3 of each, with their gamma or u), RMSNorm's strided partials are read
// back from an LDS copy of the row (thread t: x[t], x[t+256], ... in order,
// as block_rms_scale sums them), and each block is quantized from registers.
// Same operations and outputs as k_quant_batch.
template <int MAXB>
__global__ void __launch_bounds__(256) k_quant_batch_r(const float* __restrict__ x, const float* __restrict__ u,
                                                       int ld_x, const float* __restrict__ gamma, float eps, int dim,
                                                       int n_valid, int mode, _Float16* __restrict__ xh,
                                                       float* __restrict__ xd, _Float16* __restrict__ xbs) {
  __shared__ float red[260];
  __shared__ __attribute__((aligned(16))) float sx[4 * MAXB * QK_K];
  const int t = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const float* xt = x + static_cast<size_t>(t) * ld_x;
  const float* ut = u ? u + static_cast<size_t>(t) * ld_x : nullptr;
  const bool norm = (mode == PRO_NORM_AWAY || mode == PRO_NORM_EVEN);
  const bool swiglu = mode == QB_SWIGLU;
  const bool away = (mode == PRO_QUANT_AWAY || mode == PRO_NORM_AWAY || swiglu);
  const int nb = dim / QK_K;
  // x (or g), and gamma (or u); blocks past nb re-read the last, and values
  // at or past n_valid (a multiple of 4, checked by the launch; they
  // quantize as 0) read the last valid four, unused
  f32x4 xv[MAXB], wv[MAXB];
#pragma unroll
  for (int j = 0; j < MAXB; ++j) {
    const int i = min(min(wave + 4 * j, nb - 1) * QK_K + 4 * lane, n_valid - 4);
    xv[j] = *reinterpret_cast<const f32x4*>(xt + i);
    if (norm) wv[j] = *reinterpret_cast<const f32x4*>(gamma + i);
    if (swiglu) wv[j] = *reinterpret_cast<const f32x4*>(ut + i);
  }
  float rms = 1.0f;
  if (norm) {
#pragma unroll
    for (int j = 0; j < MAXB; ++j)
      if (wave + 4 * j < nb) *reinterpret_cast<f32x4*>(&sx[(wave + 4 * j) * QK_K + 4 * lane]) = xv[j];
    __syncthreads();
    float p = 0.0f;
    for (int k = 0; k < nb; ++k) {
      const float v = sx[k * QK_K + tid];
      p = p + v * v;
    }
    rms = block_rms_1sync(p, dim, eps, red);
  }
#pragma unroll
  for (int j = 0; j < MAXB; ++j) {
    const int b = wave + 4 * j;
    if (b >= nb) break;
    float v[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
    const float w4[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (swiglu) {
        const int i = b * QK_K + 4 * lane + k;
        float h = 0.0f;
        if (i < n_valid) {
          const float g = v[k];
          const float silu = g / (1.0f + exp_f32(-g));
          h = silu * w4[k];
        }
        v[k] = h;
      } else {
        if (norm) v[k] = (v[k] * rms) * w4[k];
        if (b * QK_K + 4 * lane + k >= n_valid) v[k] = 0.0f;
      }
    }
    uint32_t packed;
    float d;
    int gsum;
    quant_block_wave(v, away, packed, d, gsum);
    _Float16* o = xh + static_cast<size_t>(t) * dim + b * QK_K + 4 * lane;
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    h4 hv;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      hv[k] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>((packed >> (8 * k)) & 0xffu)));
    *reinterpret_cast<h4*>(o) = hv;
    if ((lane & 3) == 0) xbs[(static_cast<size_t>(t) * nb + b) * 16 + (lane >> 2)] = static_cast<_Float16>(gsum);
    if (lane == 0) xd[static_cast<size_t>(t) * nb + b] = d;
  }
}

// ------------------------------------------------------------------ GEMM ----
struct GemmArgs {
  WView w;
  int rows, nb, n_tok;
  const _Float16* xh;   // [n_tok][nb*256] activation codes
  const float* xd;      // [n_tok][nb] Q8_K d
  const _Float16* xbs;  // [n_tok][nb][16] bsums
  float* out;           // out[t*ld_out + r]
  int ld_out;
  int add;              // 1: out += v (residual), 0: out = v
  // an optional second matrix of the same type and blocks per row on the
  // same activations (rows2 > 0, rows a multiple of 64): the launch's rows
  // rows .. rows+rows2-1 are its rows, written to out2 (row stride ld_out2)
  WView w2;
  int rows2;
  float* out2;
  int ld_out2;
  // rope != nullptr: every row pair (2i, 2i+1) of a matrix is rotated as
  // apply_rope does before it is stored (head_dim rope_hd, token t at
  // position pos0 + t, table rows of rope_hd/2 (cos, sin) pairs)
  const float2* rope;
  int rope_hd, pos0;
  // swiglu: the two matrices are gate and up (rows2 == rows, rows % 32 ==
  // 0); a work group takes 32 rows of each (waves 0, 1: gate; 2, 3: up) and
  // writes h = silu(gate)*up (decode's gate/up epilogue) to out
  int swiglu;
};

__device__ __forceinline__ uint32_t h2bits(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// A raw buffer resource over p (byte offsets up to 2 GB).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t gemm_rsrc(const void* p) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), static_cast<short>(0), 0x7fffffff, 0x00020000);
}

// fp16 pair (1024 + byte) from bytes of t picked by sel (0x64 high bytes),
// minus off: small integers, exact
__device__ __forceinline__ h2 byte_pair_h(uint32_t t, uint32_t sel, h2 off) {
  return __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, t, sel)) - off;
}
constexpr uint32_t SEL01 = 0x04010400u, SEL23 = 0x04030402u;

// Eight halves of lane m's A operand: the low (j < 4) and high (j >= 4)
// K-halves, each four bytes of ta / tb times sa / sb, as (1024 + byte) * s +
// m in one packed fma with m = -1024 * s, whose single rounding meets the
// exact product byte * s.  Q4_K: s = sc <= 63 (m exact in fp16, byte * s <=
// 945).  Q6_K: s = sc / 64 for signed sc (m = -16 * sc, |byte * sc| <= 1920,
// so byte * sc / 64 is exact in fp16); its MFMA sums come out divided by 64,
// exactly, and the chain's scale carries the 64 back.
__device__ __forceinline__ h2 byte_pair_fma(uint32_t t, uint32_t sel, h2 s, h2 ms) {
  return __builtin_elementwise_fma(__builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, t, sel)), s, ms);
}
__device__ __forceinline__ h8 a_operand_fma(uint32_t ta, uint32_t tb, h2 sa, h2 sb, h2 ma, h2 mb) {
  const u32x4 r{h2bits(byte_pair_fma(ta, SEL01, sa, ma)), h2bits(byte_pair_fma(ta, SEL23, sa, ma)),
                h2bits(byte_pair_fma(tb, SEL01, sb, mb)), h2bits(byte_pair_fma(tb, SEL23, sb, mb))};
  return __builtin_bit_cast(h8, r);
}

__device__ __forceinline__ h2 splat_h(int v) {
  const _Float16 h = static_cast<_Float16>(static_cast<float>(v));
  return h2{h, h};
}

// A work group takes 64 rows (one 16-row tile per wave) x 16*NT tokens over
// all blocks.  The tokens' activations of a block (codes, d, bsums) are
// staged in LDS once for the four waves, double-buffered: block b+1's loads
// are in flight while block b's MFMAs run.  MFMA operand
// layout (v_mfma_f32_16x16x32_f16): lane l feeds A row l%16 and B column
// l%16 with K = 8*(l/16) .. +7; D lane l register i is row 4*(l/16)+i,
// column l%16.  With K index k = 4*s + i over sub-blocks s and bytes i,
// lane l's K range is sub-blocks 2g and 2g+1 (g = l/16): element 64g + 4m + i
// (low) and 64g + 32 + 4m + i (high) of the block for lane group m.
template <int WT, int NT, int OCC>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(OCC, 8))) k_gemm_q8k(const GemmArgs a) {
  constexpr int TOK = 16 * NT;        // tokens of the work group's tile
  constexpr int BROW = QK_K + 8;      // halves per token row of sB (padded: rows 132 dwords apart)
  // halves per token of sBs.  Q4_K: the 16 bsums (rows 12 dwords apart).
  // Q6_K: eight 16-byte records, record m = (bsums 2m, 2m+1 as an fp16
  // pair, then zeros): lane group m's offset B operand read whole; a zero
  // row after the tokens serves the lanes whose K entries are all zero.
  constexpr int BSROW = WT == 0 ? 24 : 64;
  constexpr int BSZERO = WT == 0 ? 0 : 64;
  constexpr int PPT = TOK * 32 / 256; // 16-byte pieces of a block's codes per thread
  __shared__ __attribute__((aligned(16))) _Float16 sB[2][TOK * BROW];
  __shared__ float sXd[2][TOK];
  __shared__ __attribute__((aligned(16))) _Float16 sBs[2][TOK * BSROW + BSZERO];
  const int tid = threadIdx.x, wave = tid >> 6;
  const int lane = tid & 63, g = lane >> 4, c16 = lane & 15;
  const int n_rt = (a.rows + a.rows2 + 15) >> 4;
  const int n_rg = (n_rt + 3) >> 2;
  // XCD-aware tiles: work group b runs on XCD b % 8.  Of n_rg = 8q + r row
  // groups, XCD x takes rg = x + 8j (j < q) for every token tile (token
  // tiles outer, so the tile's activations serve its q row groups from one
  // L2), and then an equal share of the r remaining row groups' (row group,
  // token tile) items, so every XCD has the same work; each XCD's L2 keeps
  // about one eighth of the matrix for the whole launch.
  const int xcd = static_cast<int>(blockIdx.x) & 7, loc = static_cast<int>(blockIdx.x) >> 3;
  const int n_tg = (a.n_tok + TOK - 1) / TOK;
  const int rq = n_rg >> 3, rr = n_rg & 7;
  const int share = (rr * n_tg + 7) >> 3;
  int rg, tg;
  if (loc < rq * n_tg) {
    rg = xcd + 8 * (loc % rq);
    tg = loc / rq;
  } else {
    const int li = xcd * share + (loc - rq * n_tg);
    if (li >= rr * n_tg) return;  // uniform in the work group, before any barrier
    rg = 8 * rq + li / n_tg;
    tg = li % n_tg;
  }
  // the work group's matrix (its 64 rows lie in one: the first has a
  // multiple of 64 rows)
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const bool second = a.swiglu ? wv >= 2 : a.rows2 > 0 && 64 * rg >= a.rows;
  const WView W = second ? a.w2 : a.w;
  const int rows = second ? a.rows2 : a.rows;
  float* const out = second ? a.out2 : a.out;
  const int ld_out = second ? a.ld_out2 : a.ld_out;
  const int r0 = a.swiglu ? 32 * rg + 16 * (wv & 1) : (4 * rg + wave) * 16 - (second ? a.rows : 0), t0 = tg * TOK;
  const bool live = r0 < rows;  // uniform in the wave: a wave past the rows only stages
  const int ra = min(r0 + c16, rows - 1);  // A operand row of this lane
  const int K = a.nb * QK_K;

  // staging of block b: piece p = tid + 256k is 16 bytes (p % 32) of token
  // p / 32's codes; thread t < TOK also takes token t's d, t < 2*TOK half of
  // token t/2's bsums.  Tokens past the end re-read the last one (unused).
  u32x4 pf[PPT], pbs;
  float pxd = 0.0f;
  // Every load of the block loop is a buffer load: the lane's byte offset is
  // the same for every block (computed once here) and the block's part is a
  // scalar offset, so the loop spends no vector instructions on addresses.
  // (Every buffer here is far below 2 GB; indices are clamped as before.)
  const __amdgpu_buffer_rsrc_t rxh = gemm_rsrc(a.xh), rxd = gemm_rsrc(a.xd), rxbs = gemm_rsrc(a.xbs);
  uint32_t vo_pf[PPT];
#pragma unroll
  for (int k = 0; k < PPT; ++k) {
    const int p = tid + 256 * k;
    const uint32_t tk = static_cast<uint32_t>(min(t0 + p / 32, a.n_tok - 1));
    vo_pf[k] = (tk * static_cast<uint32_t>(K) + static_cast<uint32_t>(p % 32) * 8) * 2;
  }
  // every thread loads (threads past the d and bsums slots re-read the
  // last slot's, unused): no branch among the loads, so the waits for them
  // count exactly
  const int td = min(tid, TOK - 1), tb = min(tid, 2 * TOK - 1);
  const uint32_t vo_xd = static_cast<uint32_t>(min(t0 + td, a.n_tok - 1)) * static_cast<uint32_t>(a.nb) * 4;
  const uint32_t vo_xbs =
      (static_cast<uint32_t>(min(t0 + tb / 2, a.n_tok - 1)) * static_cast<uint32_t>(a.nb) * 16 + (tb & 1) * 8) * 2;
  auto fetch = [&](int b) {
#pragma unroll
    for (int k = 0; k < PPT; ++k)
      pf[k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rxh, vo_pf[k], b * QK_K * 2, 0));
    pxd = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rxd, vo_xd, b * 4, 0));
    pbs = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rxbs, vo_xbs, b * 32, 0));
  };
  // sB keeps each token's 256 codes as 32 quads of 8 halves, quad 8g + m =
  // elements 64g + 4m .. +3 and 64g + 32 + 4m .. +3 (the B operand of lane
  // group m for the lanes of K-half g), stored at slot (8g + m) ^ sw(g) with
  // sw = 0, 1, 1, 0 for g = 0..3: the lanes of one pass of 8-byte stores (16
  // or 32) then write distinct banks, where unswapped quads 8 and 16 apart
  // share them.  Piece k = p % 32 (elements 8k .. 8k+7, g = k/8, h =
  // (k/4)%2, m = 2*(k%4)) goes to half h of quads m, m+1.
  auto stash = [&](int buf) {
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int p = tid + 256 * k;
      const int pk = p % 32, gq = pk >> 3, hq = (pk >> 2) & 1, mq = 2 * (pk & 3), sw = (gq ^ (gq >> 1)) & 1;
      _Float16* row = &sB[buf][(p / 32) * BROW + 4 * hq];
      *reinterpret_cast<uint2*>(row + ((8 * gq + mq) ^ sw) * 8) = uint2{pf[k].x, pf[k].y};
      *reinterpret_cast<uint2*>(row + ((8 * gq + mq + 1) ^ sw) * 8) = uint2{pf[k].z, pf[k].w};
    }
    if (tid < TOK) sXd[buf][tid] = pxd;
    if (tid < 2 * TOK) {
      if constexpr (WT == 0) {
        *reinterpret_cast<u32x4*>(&sBs[buf][(tid / 2) * BSROW + (tid & 1) * 8]) = pbs;
      } else {
        const uint32_t pw[4] = {pbs.x, pbs.y, pbs.z, pbs.w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *reinterpret_cast<uint32_t*>(&sBs[buf][(tid / 2) * BSROW + (4 * (tid & 1) + j) * 8]) = pw[j];
      }
    }
  };
  if constexpr (WT == 1) {
    // the records' zero dwords and the zero row, written once (the stash
    // writes only the pairs)
    for (int i = tid; i < 2 * (TOK * BSROW + BSZERO) / 8; i += 256)
      reinterpret_cast<u32x4*>(&sBs[0][0])[i] = u32x4{0u, 0u, 0u, 0u};
    __syncthreads();
  }
  fetch(0);
  stash(0);
  __syncthreads();

  float acc[NT][8][4], accm[NT][4];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      accm[n][i] = 0.0f;
#pragma unroll
      for (int m = 0; m < 8; ++m) acc[n][m][i] = 0.0f;
    }
  }
  const h2 off1024{static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
  const h2 q4c16{static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
  const h2 q4cm64{static_cast<_Float16>(-64.0f), static_cast<_Float16>(-64.0f)};
  const h2 q4cm1024{static_cast<_Float16>(-1024.0f), static_cast<_Float16>(-1024.0f)};
  const f32x4 zero4{0.0f, 0.0f, 0.0f, 0.0f};
  // Q6_K, per lane (K-half g: code fields at bit 4*(g&1) of each byte, and
  // the high bits' second field 2 above): field masks and the constants of
  // the scale builds (f = 2^-p for a field at bit p)
  struct Q6Consts {
    uint32_t ml, ma0, ma1;
    h2 sl1, sl2, ol1, ol2, sa1, sa2, oa1, oa2, c1, c2;
  };
  const Q6Consts q6c = [&] {
    const bool odd = (g & 1) != 0;
    const float fl = odd ? 0.0625f : 1.0f, fa = odd ? 0.015625f : 0.25f;
    auto hs = [](float v) {
      const _Float16 h = static_cast<_Float16>(v);
      return h2{h, h};
    };
    return Q6Consts{odd ? 0xf0f0f0f0u : 0x0f0f0f0fu, odd ? 0x30303030u : 0x03030303u, odd ? 0xc0c0c0c0u : 0x0c0c0c0cu,
                    hs(fl * 0.015625f), hs(-18.0f * fl), hs(-16.0f * fl), hs(18432.0f * fl),
                    hs(fa * 0.015625f), hs(-18.0f * fa), hs(-16.0f * fa), hs(18432.0f * fa),
                    hs(-0.03125f), hs(36.0f)};
  }();

  // The weight bytes a block's A operands and row scales are built from,
  // loaded one block ahead like the activations (loaded in their own block,
  // they would hold every block's MFMAs for a full memory round trip).
  // Q4_K: hdr = the A row's d/dmin/scales, q[0..1] = its chunk planes 2g and
  // 2g+1; Q6_K: hdr = its scales, q[0..3] = ql planes 4h.., q[4..5] = qh
  // planes 2h..; dr[i] = d (and Q4_K's dmin) of D row 4g+i.
  // (Q4_K's hdr is the 12 scale bytes only: a dword of a vector load left
  // unused is a register the compiler reuses, and reusing it waits for every
  // load in flight)
  struct WRaw {
    typename std::conditional<WT == 0, u32x3, u32x4>::type hdr;
    u32x4 q[WT == 0 ? 2 : 6];
    uint32_t dr[4];
  };
  const __amdgpu_buffer_rsrc_t rw0 = gemm_rsrc(W.p0), rw1 = gemm_rsrc(W.p1), rw2 = gemm_rsrc(W.p2),
                               rw3 = gemm_rsrc(W.p3);
  const uint32_t rows16 = static_cast<uint32_t>(rows) * 16;
  uint32_t vo_dr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    vo_dr[i] = static_cast<uint32_t>(min(r0 + 4 * g + i, rows - 1)) * (WT == 0 ? 16u : 2u);
  const uint32_t vo_ra = static_cast<uint32_t>(ra) * 16;
  auto load_w = [&](WRaw& w, int b) {
    const uint32_t ub = static_cast<uint32_t>(b);
    if constexpr (WT == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) w.dr[i] = __builtin_amdgcn_raw_buffer_load_b32(rw1, vo_dr[i], ub * rows16, 0);
      w.hdr = __builtin_bit_cast(u32x3, __builtin_amdgcn_raw_buffer_load_b96(rw1, vo_ra + 4, ub * rows16, 0));
#pragma unroll
      for (int j = 0; j < 2; ++j)
        w.q[j] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw0, vo_ra + (2 * g + j) * rows16, ub * 8 * rows16, 0));
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w.dr[i] = __builtin_amdgcn_raw_buffer_load_b16(rw3, vo_dr[i], ub * static_cast<uint32_t>(rows) * 2, 0);
      const int h = g >> 1;
      w.hdr = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw2, vo_ra, ub * rows16, 0));
#pragma unroll
      for (int cc = 0; cc < 4; ++cc)
        w.q[cc] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw0, vo_ra + (4 * h + cc) * rows16, ub * 8 * rows16, 0));
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
        w.q[4 + cc] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw1, vo_ra + (2 * h + cc) * rows16, ub * 4 * rows16, 0));
    }
  };
  // One block: the weight bytes of block b+1 (into nxt) and its activations
  // are loaded while block b's MFMAs run; cur and nxt trade places each
  // block, so no copy waits for loads in flight.
  auto block = [&](int b, const WRaw& wc, WRaw& wn) {
    const int buf = b & 1;
    // in flight during this block's MFMAs; issued unconditionally (the last
    // block loads itself again, unused), so the wait for wc's loads counts
    // the same number of younger loads on every path and leaves these in
    // flight
    const int bn = min(b + 1, a.nb - 1);
    fetch(bn);
    load_w(wn, bn);
    if (live) {
    // d (and dmin) of the four D rows of this lane
    float dw[4], dmw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (WT == 0) {
        dw[i] = fp16_to_fp32(static_cast<uint16_t>(wc.dr[i] & 0xffffu));
        dmw[i] = fp16_to_fp32(static_cast<uint16_t>(wc.dr[i] >> 16));
      } else {
        dw[i] = fp16_to_fp32(static_cast<uint16_t>(wc.dr[i]));
        dmw[i] = 0.0f;
      }
    }
    // Lane groups in order; each one's A operand is built from the weight
    // bytes just before its MFMAs (one per token tile, the operand then
    // dropped), so the build of the next overlaps them.
    float ds[NT][4], xdv[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      xdv[n] = sXd[buf][16 * n + c16];
#pragma unroll
      for (int i = 0; i < 4; ++i) ds[n][i] = WT == 0 ? xdv[n] * dw[i] : (xdv[n] * dw[i]) * 64.0f;
    }
    // the B operand of lane group m for token tile n is quad 8g + m of the
    // token's row (at slot (8g + m) ^ sw(g))
    auto bq = [&](int n, int m) {
      return __builtin_bit_cast(h8, reinterpret_cast<const u32x4*>(&sB[buf][(16 * n + c16) * BROW])[(8 * g + m) ^ ((g ^ (g >> 1)) & 1)]);
    };
    if constexpr (WT == 0) {
      const uint32_t s0 = wc.hdr.x, s1 = wc.hdr.y, s2 = wc.hdr.z;
      const uint32_t sc_lo = s0 & 0x3f3f3f3fu;
      const uint32_t sc_hi = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
      const uint32_t mn_lo = s1 & 0x3f3f3f3fu;
      const uint32_t mn_hi = ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u);
      // sc[2g] (low nibbles) and sc[2g+1]/16 (high nibbles, read in place as
      // 16*code), from fp16 (1024 + sc) by byte permute; the offsets -1024*s
      // (exact: sc <= 63)
      const uint32_t sw = g < 2 ? sc_lo : sc_hi;
      const uint32_t bs = 2 * (g & 1);
      const h2 ha = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, sw, 0x04000400u | (bs << 16) | bs));
      const h2 hb = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, sw, 0x04000400u | ((bs + 1) << 16) | (bs + 1)));
      const h2 sa = ha - off1024, sb = __builtin_elementwise_fma(hb, q4c16, q4cm64);
      const h2 ma = sa * q4cm1024, mb = sb * q4cm1024;
      const u32x4 q0 = wc.q[0], q1 = wc.q[1];
      const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
      // two lane groups at a time: their 2*NT MFMAs are independent and
      // issue back to back before the first chain step reads a result; the
      // next pair's B operands are read from LDS while this pair's run
      h8 Bc[2][NT];
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        Bc[0][n] = bq(n, 0);
        Bc[1][n] = bq(n, 1);
      }
#pragma unroll
      for (int m = 0; m < 8; m += 2) {
        h8 Bn[2][NT];
        if (m + 2 < 8) {
#pragma unroll
          for (int n = 0; n < NT; ++n) {
            Bn[0][n] = bq(n, m + 2);
            Bn[1][n] = bq(n, m + 3);
          }
        }
        const h8 A0 = a_operand_fma(qw[m] & 0x0f0f0f0fu, qw[m] & 0xf0f0f0f0u, sa, sb, ma, mb);
        const h8 A1 = a_operand_fma(qw[m + 1] & 0x0f0f0f0fu, qw[m + 1] & 0xf0f0f0f0u, sa, sb, ma, mb);
        f32x4 D0[NT], D1[NT];
#pragma unroll
        for (int n = 0; n < NT; ++n) {
          D0[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, Bc[0][n], zero4, 0, 0, 0);
          D1[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, Bc[1][n], zero4, 0, 0, 0);
        }
        if (m + 2 < 8) {
#pragma unroll
          for (int n = 0; n < NT; ++n) {
            Bc[0][n] = Bn[0][n];
            Bc[1][n] = Bn[1][n];
          }
        }
#pragma unroll
        for (int n = 0; n < NT; ++n) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc[n][m][i] = __builtin_fmaf(ds[n][i], D0[n][i], acc[n][m][i]);
            acc[n][m + 1][i] = __builtin_fmaf(ds[n][i], D1[n][i], acc[n][m + 1][i]);
          }
        }
      }
      // min operand: k = 8g + j < 16 -> mn[k/2]
      const uint32_t mw = (g & 1) ? mn_hi : mn_lo;
      const u32x4 mr{h2bits(byte_pair_h(mw, 0x04000400u, off1024)), h2bits(byte_pair_h(mw, 0x04010401u, off1024)),
                     h2bits(byte_pair_h(mw, 0x04020402u, off1024)), h2bits(byte_pair_h(mw, 0x04030403u, off1024))};
      const h8 AM = g < 2 ? __builtin_bit_cast(h8, mr) : h8{};
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        const h8 BM = *reinterpret_cast<const h8*>(&sBs[buf][(16 * n + c16) * BSROW + 8 * (g & 1)]);
        const f32x4 DM = __builtin_amdgcn_mfma_f32_16x16x32_f16(AM, BM, zero4, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) accm[n][i] = __builtin_fmaf(-(xdv[n] * dmw[i]), DM[i], accm[n][i]);
      }
    } else {
      // The 16 scales as unsigned bytes u = sc + 128; fp16 (1024 + u) from a
      // byte permute, then one packed fma gives sc*f/64 = (1024 + u)*f/64 -
      // 18*f or -16*sc*f = (1024 + u)*(-16*f) + 18432*f, exactly (f a power of
      // two).  The lane's code fields are masked in place (not shifted): a
      // field at bit p of its byte reads as code*2^p, and its scale carries
      // f = 2^-p, so every A entry is still code*sc/64.
      const u32x4 scr = wc.hdr;
      const uint32_t su[4] = {scr.x ^ 0x80808080u, scr.y ^ 0x80808080u, scr.z ^ 0x80808080u, scr.w ^ 0x80808080u};
      const uint32_t scw = g == 0 ? su[0] : g == 1 ? su[1] : g == 2 ? su[2] : su[3];  // scales 4g .. 4g+3
      h2 sL[4], oL[4], sA[2], oA[2];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const h2 hb = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, scw, 0x04000400u | (k << 16) | k));
        sL[k] = __builtin_elementwise_fma(hb, q6c.sl1, q6c.sl2);
        oL[k] = __builtin_elementwise_fma(hb, q6c.ol1, q6c.ol2);
        if (k >= 2) {
          sA[k - 2] = __builtin_elementwise_fma(hb, q6c.sa1, q6c.sa2);
          oA[k - 2] = __builtin_elementwise_fma(hb, q6c.oa1, q6c.oa2);
        }
      }
      uint32_t lw[16], hw[8];
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        const u32x4 v = wc.q[cc];
        lw[4 * cc] = v.x;
        lw[4 * cc + 1] = v.y;
        lw[4 * cc + 2] = v.z;
        lw[4 * cc + 3] = v.w;
      }
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        const u32x4 v = wc.q[4 + cc];
        hw[4 * cc] = v.x;
        hw[4 * cc + 1] = v.y;
        hw[4 * cc + 2] = v.z;
        hw[4 * cc + 3] = v.w;
      }
      // one lane group's operands; two lane groups' MFMAs are issued before
      // either chain reads a result
      auto q6_ops = [&](int m, h8& Al, h8& Ah, uint32_t& AC) {
        const int ka = m >> 2, kb = 2 + (m >> 2);
        Al = a_operand_fma(lw[m] & q6c.ml, lw[8 + m] & q6c.ml, sL[ka], sL[kb], oL[ka], oL[kb]);
        Ah = a_operand_fma(hw[m] & q6c.ma0, hw[m] & q6c.ma1, sL[ka], sA[kb - 2], oL[ka], oA[kb - 2]);
        // the offset operand's first K pair: -2*sc[2m]/64, -2*sc[2m+1]/64 of
        // this lane's row (-sc/32 = (1024 + u)*(-1/32) + 36)
        const uint32_t sel = 0x04000400u | ((2 * (m & 1) + 1) << 16) | (2 * (m & 1));
        const h2 hp = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, su[m >> 1], sel));
        AC = h2bits(__builtin_elementwise_fma(hp, q6c.c1, q6c.c2));
      };
      // S + 16*T for lane group m and token tile n: S = sc*ql*x, T = sc*qh*x - 2C
      // (each divided by 64, exactly)
      // the B operand and the bsums pair of lane group m, token tile n
      struct BOp {
        h8 B;
        h8 BC;  // record m of the token (lanes 0..15), the zero row (the others)
      };
      auto b_op = [&](int m, int n) {
        const int row = g == 0 ? (16 * n + c16) * BSROW : TOK * BSROW;
        return BOp{bq(n, m), *reinterpret_cast<const h8*>(&sBs[buf][row + m * 8])};
      };
      // The offset operand is Al with its first dword replaced by the pair
      // (formed after the S MFMAs have read Al): its other K entries meet
      // zeros of BC, and lanes 16..63 read an all-zero BC, so NC is the
      // offset alone.
      auto q6_mfma = [&](const BOp& o, const h8& Al, const h8& Ah, uint32_t AC, f32x4& S, f32x4& T) {
        S = __builtin_amdgcn_mfma_f32_16x16x32_f16(Al, o.B, zero4, 0, 0, 0);
        const u32x4 al = __builtin_bit_cast(u32x4, Al);
        const h8 A2 = __builtin_bit_cast(h8, u32x4{AC, al.y, al.z, al.w});
        const f32x4 NC = __builtin_amdgcn_mfma_f32_16x16x32_f16(A2, o.BC, zero4, 0, 0, 0);  // -2C
        T = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ah, o.B, NC, 0, 0, 0);
      };
      // Lane groups in steps of LG: pairs with one token tile (their six
      // MFMAs independent), one at a time with two (registers: two tiles'
      // accumulators, sums and B operands).  The next step's B operands are
      // read from LDS while this step's MFMAs run.
      constexpr int LG = NT >= 2 ? 1 : 2;
      BOp Oc[LG][NT];
#pragma unroll
      for (int j = 0; j < LG; ++j) {
#pragma unroll
        for (int n = 0; n < NT; ++n) Oc[j][n] = b_op(j, n);
      }
#pragma unroll
      for (int m = 0; m < 8; m += LG) {
        BOp On[LG][NT];
        if (m + LG < 8) {
#pragma unroll
          for (int j = 0; j < LG; ++j) {
#pragma unroll
            for (int n = 0; n < NT; ++n) On[j][n] = b_op(m + LG + j, n);
          }
        }
        h8 Al[LG], Ah[LG];
        uint32_t AC[LG];
#pragma unroll
        for (int j = 0; j < LG; ++j) q6_ops(m + j, Al[j], Ah[j], AC[j]);
        f32x4 S[LG][NT], T[LG][NT];
#pragma unroll
        for (int n = 0; n < NT; ++n) {
#pragma unroll
          for (int j = 0; j < LG; ++j) q6_mfma(Oc[j][n], Al[j], Ah[j], AC[j], S[j][n], T[j][n]);
        }
        if (m + LG < 8) {
#pragma unroll
          for (int j = 0; j < LG; ++j) {
#pragma unroll
            for (int n = 0; n < NT; ++n) Oc[j][n] = On[j][n];
          }
        }
#pragma unroll
        for (int n = 0; n < NT; ++n) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int j = 0; j < LG; ++j)
              acc[n][m + j][i] = __builtin_fmaf(ds[n][i], __builtin_fmaf(16.0f, T[j][n][i], S[j][n][i]), acc[n][m + j][i]);
          }
        }
      }
    }
    }  // live
    // block b+1 into the other buffer, whose last readers passed the previous
    // barrier (after the last block: a copy of it, never read)
    stash(buf ^ 1);
    __syncthreads();
  };
  WRaw w0, w1;
  load_w(w0, 0);
  // pairs of blocks with no branch inside, then the odd block
  int b = 0;
  for (; b + 1 < a.nb; b += 2) {
    block(b, w0, w1);
    block(b + 1, w1, w0);
  }
  if (b < a.nb) block(b, w0, w1);

  float vs[NT][4];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      vs[n][i] = ((acc[n][0][i] + acc[n][4][i]) + (acc[n][2][i] + acc[n][6][i])) +
                 ((acc[n][1][i] + acc[n][5][i]) + (acc[n][3][i] + acc[n][7][i]));
      if constexpr (WT == 0) vs[n][i] = vs[n][i] + accm[n][i];
    }
  }
  if (a.swiglu) {
    // the up waves hand their values to the gate waves of the same rows and
    // tokens through LDS (sB is free: every read of it passed the last
    // block's barrier)
    float* xs = reinterpret_cast<float*>(&sB[0][0]);
    if (second) {
#pragma unroll
      for (int n = 0; n < NT; ++n) {
#pragma unroll
        for (int i = 0; i < 4; ++i) xs[(((wv & 1) * NT + n) * 4 + i) * 64 + lane] = vs[n][i];
      }
    }
    __syncthreads();
    if (second) return;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float gv = vs[n][i], uv = xs[(((wv & 1) * NT + n) * 4 + i) * 64 + lane];
        vs[n][i] = (gv / (1.0f + exp_f32(-gv))) * uv;
      }
    }
  }
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int t = t0 + 16 * n + c16;
    float v[4] = {vs[n][0], vs[n][1], vs[n][2], vs[n][3]};
    if (a.rope) {
      // rows 4g+i of the lane: pairs (0, 1) and (2, 3), apply_rope's
      // products and sums (src/ops/ops.cpp:502-516)
      const size_t pos = static_cast<size_t>(a.pos0 + min(t, a.n_tok - 1));
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        const int d = (r0 + 4 * g + i) % a.rope_hd;
        const float2 cs = a.rope[pos * (a.rope_hd / 2) + (d >> 1)];
        const float e = v[i], o = v[i + 1];
        v[i] = e * cs.x - o * cs.y;
        v[i + 1] = e * cs.y + o * cs.x;
      }
    }
    // the lane's four rows are consecutive: one 16-byte access where all
    // four exist and the address is aligned, else one by one
    const int r4 = r0 + 4 * g;
    float* o = out + static_cast<size_t>(min(t, a.n_tok - 1)) * ld_out + r4;
    if (t < a.n_tok) {
      if (r4 + 3 < rows && (reinterpret_cast<uintptr_t>(o) & 15) == 0) {
        f32x4 w{v[0], v[1], v[2], v[3]};
        if (a.add) {
          const f32x4 p = *reinterpret_cast<const f32x4*>(o);
          w = f32x4{p.x + v[0], p.y + v[1], p.z + v[2], p.w + v[3]};
        }
        *reinterpret_cast<f32x4*>(o) = w;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (r4 + i < rows) o[i] = a.add ? o[i] + v[i] : v[i];
      }
    }
  }
}

// ------------------------------------------------- attention combine + Q8_K --
// Per token t (one work group, position pos0 + t): the attention output from
// the per-token chunk partials -- k_attn_combine's arithmetic for each value:
// m = max m_c, then over the chunks in order f_c = exp(m_c - m),
// Z = fma(z_c, f_c, Z), O = fma(o_c, f_c, O), value O / Z -- then the O
// projection's ties-even Q8_K quantization of it (k_quant_batch's), with no
// fp32 copy of the output in between.  A lane takes 4 consecutive values of
// one head (head_dim % 4 == 0), which share m and Z.
__global__ void __launch_bounds__(256) k_quant_batch_attn(const float* __restrict__ part_o,
                                                          const float2* __restrict__ part_mz, size_t tok_stride_o,
                                                          size_t tok_stride_mz, int pos0, int dim, int hd,
                                                          int max_chunks, _Float16* __restrict__ xh,
                                                          float* __restrict__ xd, _Float16* __restrict__ xbs) {
  const int t = blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nch = (pos0 + t) / ATTN_CHUNK + 1;
  const int nb = dim / QK_K;
  for (int b = wave; b < nb; b += 4) {
    const int i0 = b * QK_K + 4 * lane;
    const int h = i0 / hd, d0 = i0 - h * hd;
    const float2* mz = part_mz + t * tok_stride_mz + static_cast<size_t>(h) * max_chunks;
    const float* o = part_o + t * tok_stride_o + static_cast<size_t>(h) * max_chunks * hd + d0;
    // the chunks' partials in batches of CB whose loads are issued together
    // (indices past the last chunk re-read it: the max is unchanged, and the
    // combine skips them)
    constexpr int CB = 8;
    float m = mz[0].x;
    for (int c0 = 0; c0 < nch; c0 += CB) {
      float mv[CB];
#pragma unroll
      for (int k = 0; k < CB; ++k) mv[k] = mz[min(c0 + k, nch - 1)].x;
#pragma unroll
      for (int k = 0; k < CB; ++k) m = fmaxf(m, mv[k]);
    }
    float Z = 0.0f;
    float O[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int c0 = 0; c0 < nch; c0 += CB) {
      float2 zc[CB];
      f32x4 oc[CB];
#pragma unroll
      for (int k = 0; k < CB; ++k) {
        const int c = min(c0 + k, nch - 1);
        zc[k] = mz[c];
        oc[k] = *reinterpret_cast<const f32x4*>(o + static_cast<size_t>(c) * hd);
      }
#pragma unroll
      for (int k = 0; k < CB; ++k) {
        if (c0 + k < nch) {
          const float f = exp_f32(zc[k].x - m);
          Z = __builtin_fmaf(zc[k].y, f, Z);
          O[0] = __builtin_fmaf(oc[k].x, f, O[0]);
          O[1] = __builtin_fmaf(oc[k].y, f, O[1]);
          O[2] = __builtin_fmaf(oc[k].z, f, O[2]);
          O[3] = __builtin_fmaf(oc[k].w, f, O[3]);
        }
      }
    }
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = O[k] / Z;
    uint32_t packed;
    float dq;
    int gsum;
    quant_block_wave(v, false, packed, dq, gsum);
    _Float16* out = xh + static_cast<size_t>(t) * dim + i0;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      out[k] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>((packed >> (8 * k)) & 0xffu)));
    if ((lane & 3) == 0) xbs[(static_cast<size_t>(t) * nb + b) * 16 + (lane >> 2)] = static_cast<_Float16>(gsum);
    if (lane == 0) xd[static_cast<size_t>(t) * nb + b] = dq;
  }
}

// -------------------------------------------------------------- launchers --
hipError_t launch_embed_batch(const WView& w, const int* tokens, int n_tok, int dim, float* x, hipStream_t s) {
  hipLaunchKernelGGL(k_embed_batch, dim3((dim + QK_K - 1) / QK_K, n_tok), dim3(QK_K), 0, s, w, tokens, dim, x);
  return hipGetLastError();
}

hipError_t launch_quant_batch(const float* x, const float* u, int ld_x, const float* gamma, float eps, int dim,
                              int n_valid, int mode, int n_tok, QuantBatch q, hipStream_t s) {
  if (dim % QK_K) return hipErrorInvalidValue;
  // rows of up to 24 blocks load everything up front (k_quant_batch_r)
  const int nb = dim / QK_K;
  if (n_valid < 1 || n_valid > dim || n_valid > ld_x) return hipErrorInvalidValue;
  const bool up_front = ld_x % 4 == 0 && n_valid % 4 == 0;
  if (up_front && nb <= 12)
    hipLaunchKernelGGL(k_quant_batch_r<3>, dim3(n_tok), dim3(256), 0, s, x, u, ld_x, gamma, eps, dim, n_valid, mode,
                       q.xh, q.xd, q.xbs);
  else if (up_front && nb <= 24)
    hipLaunchKernelGGL(k_quant_batch_r<6>, dim3(n_tok), dim3(256), 0, s, x, u, ld_x, gamma, eps, dim, n_valid, mode,
                       q.xh, q.xd, q.xbs);
  else
    hipLaunchKernelGGL(k_quant_batch, dim3(n_tok), dim3(256), 0, s, x, u, ld_x, gamma, eps, dim, n_valid, mode,
                       q.xh, q.xd, q.xbs);
  return hipGetLastError();
}

hipError_t launch_quant_batch_swiglu(const float* g, const float* u, int ld, int n_valid, int dim, int n_tok,
                                     QuantBatch q, hipStream_t s) {
  return launch_quant_batch(g, u, ld, nullptr, 0.0f, dim, n_valid, QB_SWIGLU, n_tok, q, s);
}

hipError_t launch_gemm_q8k(const WView& w, int rows, int nb, int n_tok, const QuantBatch& q, float* out, int ld_out,
                           bool add, hipStream_t s, const WView* w2, int rows2, float* out2, int ld_out2,
                           const GemmRope* rope, bool swiglu) {
  if (w.type != MCPM_TYPE_Q4_K && w.type != MCPM_TYPE_Q6_K) return hipErrorInvalidValue;
  if (rows2 > 0 && (!w2 || w2->type != w.type || rows % 64 || (!swiglu && !out2))) return hipErrorInvalidValue;
  if (swiglu && (rows2 != rows || rows % 32 || rope || add)) return hipErrorInvalidValue;
  // a rotated pair (rows 2i, 2i+1) stays in one head and one lane: head_dim
  // even, every matrix's rows a multiple of it
  if (rope && (!rope->table || rope->head_dim <= 0 || rope->head_dim % 2 || rows % rope->head_dim ||
               (rows2 > 0 && rows2 % rope->head_dim)))
    return hipErrorInvalidValue;
  GemmArgs a{w, rows, nb, n_tok, q.xh, q.xd, q.xbs, out, ld_out, add ? 1 : 0, rows2 > 0 ? *w2 : WView{},
             std::max(rows2, 0), out2, ld_out2, rope ? rope->table : nullptr, rope ? rope->head_dim : 0,
             rope ? rope->pos0 : 0, swiglu ? 1 : 0};
  rows += std::max(rows2, 0);
  // token tiles per wave and waves per SIMD (MCPM_PREFILL_NT=1|2|4 and
  // MCPM_PREFILL_OCC=1|2 override, tuning aids; "a,b" sets Q4_K a, Q6_K b)
  struct Pair {
    int q4 = 0, q6 = 0;
  };
  auto env_pair = [](const char* name) {
    Pair p;
    if (const char* v = std::getenv(name)) {
      const int n = std::sscanf(v, "%d,%d", &p.q4, &p.q6);
      if (n == 1) p.q6 = p.q4;
    }
    return p;
  };
  static const Pair nt_env = env_pair("MCPM_PREFILL_NT"), occ_env = env_pair("MCPM_PREFILL_OCC");
  const bool q4 = w.type == MCPM_TYPE_Q4_K;
  const int nt_e = q4 ? nt_env.q4 : nt_env.q6, occ_e = q4 ? occ_env.q4 : occ_env.q6;
  // Defaults: two waves per SIMD (registers held to 256 so a second wave hides
  // the first's load latency); 32 tokens per wave for Q4_K, 16 for Q6_K, whose
  // four MFMA operand sets need the room.
  const int NT = nt_e == 1 || nt_e == 2 || nt_e == 4 ? nt_e : (q4 ? 2 : 1);
  const int OCC = occ_e == 1 ? 1 : 2;
  // one work group per 64 rows (four 16-row tiles) x 16*NT tokens: per XCD,
  // q row groups x token tiles and a share of the other r (see k_gemm_q8k)
  const int n_rg = (rows + 63) / 64, n_tg = (n_tok + 16 * NT - 1) / (16 * NT);
  const dim3 grid(8 * ((n_rg / 8) * n_tg + ((n_rg % 8) * n_tg + 7) / 8));
#define MCPM_GEMM(N, O) \
  if (NT == N && OCC == O) { \
    if (q4) launch_kernel(k_gemm_q8k<0, N, O>, grid, dim3(256), 0, s, a); \
    else launch_kernel(k_gemm_q8k<1, N, O>, grid, dim3(256), 0, s, a); \
  }
  MCPM_GEMM(1, 1) MCPM_GEMM(1, 2) MCPM_GEMM(2, 1) MCPM_GEMM(2, 2) MCPM_GEMM(4, 1) MCPM_GEMM(4, 2)
#undef MCPM_GEMM
  return hipGetLastError();
}

hipError_t launch_quant_batch_attn(const AttnPart& part, size_t tok_stride_o, size_t tok_stride_mz, int pos0,
                                  int n_tok, int n_heads, int head_dim, int max_chunks, QuantBatch q, hipStream_t s) {
  const int dim = n_heads * head_dim;
  if (dim % QK_K || head_dim % 4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_quant_batch_attn, dim3(n_tok), dim3(256), 0, s, part.o, part.mz, tok_stride_o, tok_stride_mz,
                     pos0, dim, head_dim, max_chunks, q.xh, q.xd, q.xbs);
  return hipGetLastError();
}

}  // namespace mcpm
