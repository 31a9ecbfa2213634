// Block-level bodies of the k-quant encoder and decoder (bit-exact with
// coldpress/kquant.py), shared by the single-tensor kernels of kq_codec.hip and
// the many-tensor kernels of the EF driver.
//
// Encoder mapping: one lane per sub-block. A wave64 holds S = 64/G superblocks
// (G = 16 lanes per superblock for the 16-wide sub-blocks, 8 for the 32-wide
// ones of Q4_K and Q5_K). Sub-block fits run in-lane on registers; superblock-level
// steps (maxima, super-scale fits, the 256-wide sum of squares) run across the
// G lanes of the superblock with xor-butterfly reductions that reproduce
// numpy's pairwise order. Codes and per-superblock fields are staged in LDS
// and the wave's contiguous output bytes leave as coalesced dword stores.
#pragma once
#include <hip/hip_runtime.h>

#include "cp_device.h"
#include "cp_host.h"
#include "kq_fit.h"

namespace cp {

constexpr int kWavesPerBlock = 4;

template <int TT>
struct Kq;
template <>
struct Kq<CP_Q2_K> {
  static constexpr int G = 16, SUBW = 16, BP = 84;
};
template <>
struct Kq<CP_Q3_K> {
  static constexpr int G = 16, SUBW = 16, BP = 110;
};
template <>
struct Kq<CP_Q4_K> {
  static constexpr int G = 8, SUBW = 32, BP = 144;
};
template <>
struct Kq<CP_Q5_K> {
  static constexpr int G = 8, SUBW = 32, BP = 176;
};
template <>
struct Kq<CP_Q6_K> {
  static constexpr int G = 16, SUBW = 16, BP = 210;
};

// Per-superblock fields staged in LDS before packing.
//  Q2_K: a[k] = scale byte (sc & 0xF) | (min & 0xF) << 4
//  Q3_K: a[k] = 6-bit scale 0..63
//  Q4_K, Q5_K: a[0..7] = 6-bit scales, a[8..15] = 6-bit mins
//  Q6_K: a[k] = int8 scale
struct SbFields {
  uint8_t a[16];
  uint16_t d, dmin;
};

// numpy's pairwise sum of a superblock's 256 values staged in LDS, computed by
// the G lanes of the superblock: split 128 + 128, each half with 8 sequential
// accumulators over stride 8, then the 8-way tree (kquant.py:381, :453, :537).
template <int G>
__device__ __forceinline__ float sum256_lds(const float* a, int g) {
  if constexpr (G == 16) {
    const float* p = a + (g >> 3) * 128 + (g & 7);
    float r = p[0];
#pragma unroll
    for (int m = 1; m < 16; ++m) r = r + p[8 * m];
    r = r + __shfl_xor(r, 1);
    r = r + __shfl_xor(r, 2);
    r = r + __shfl_xor(r, 4);
    float tot = r + __shfl_xor(r, 8);
    return 0.0f + tot;
  } else {
    float r0 = a[g], r1 = a[128 + g];
#pragma unroll
    for (int m = 1; m < 16; ++m) {
      r0 = r0 + a[g + 8 * m];
      r1 = r1 + a[128 + g + 8 * m];
    }
    r0 = r0 + __shfl_xor(r0, 1);
    r1 = r1 + __shfl_xor(r1, 1);
    r0 = r0 + __shfl_xor(r0, 2);
    r1 = r1 + __shfl_xor(r1, 2);
    r0 = r0 + __shfl_xor(r0, 4);
    r1 = r1 + __shfl_xor(r1, 4);
    return 0.0f + (r0 + r1);
  }
}

// One output byte of a packed superblock from its staged codes and fields
// (ggml block layouts; kquant.py:407-413, :474-485, :565-571, :664-677).
template <int TT>
__device__ __forceinline__ uint32_t pack_byte(const uint8_t* c, const SbFields& f, int b) {
  if constexpr (TT == CP_Q2_K) {
    if (b < 16) return f.a[b];
    if (b < 80) {
      int k = b - 16, base = (k >> 5) * 128 + (k & 31);
      return c[base] | c[base + 32] << 2 | c[base + 64] << 4 | c[base + 96] << 6;
    }
    if (b < 82) return (f.d >> (8 * (b - 80))) & 0xFF;
    return (f.dmin >> (8 * (b - 82))) & 0xFF;
  } else if constexpr (TT == CP_Q3_K) {
    if (b < 32) {
      uint32_t m = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) m |= ((c[32 * j + b] >> 2) & 1u) << j;
      return m;
    }
    if (b < 96) {
      int k = b - 32, base = (k >> 5) * 128 + (k & 31);
      return (c[base] & 3) | (c[base + 32] & 3) << 2 | (c[base + 64] & 3) << 4 |
             (c[base + 96] & 3) << 6;
    }
    if (b < 108) {
      int m = b - 96;
      if (m < 8) return (f.a[m] & 0xF) | (f.a[m + 8] & 0xF) << 4;
      m -= 8;
      uint32_t v = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) v |= ((uint32_t)(f.a[m + 4 * q] >> 4) & 3u) << (2 * q);
      return v;
    }
    return (f.d >> (8 * (b - 108))) & 0xFF;
  } else if constexpr (TT == CP_Q4_K || TT == CP_Q5_K) {
    if (b < 2) return (f.d >> (8 * b)) & 0xFF;
    if (b < 4) return (f.dmin >> (8 * (b - 2))) & 0xFF;
    if (b < 16) {
      int m = b - 4;
      if (m < 4) return (f.a[m] | (f.a[m + 4] >> 4) << 6) & 0xFF;
      if (m < 8) return (f.a[8 + m - 4] | (f.a[8 + m] >> 4) << 6) & 0xFF;
      return (f.a[m - 4] & 0xF) | (f.a[8 + m - 4] & 0xF) << 4;
    }
    constexpr int body = TT == CP_Q5_K ? 48 : 16;
    if (TT == CP_Q5_K && b < body) {
      // qh: bit 2c of byte j is code (64c + j) >= 16, bit 2c+1 is code (64c + 32 + j) >= 16
      int j = b - 16;
      uint32_t v = 0;
#pragma unroll
      for (int q = 0; q < 8; ++q) v |= (uint32_t)(c[32 * q + j] >> 4) << q;
      return v;
    }
    int k = b - body, base = (k >> 5) * 64 + (k & 31);
    return (c[base] & 0xF) | (c[base + 32] & 0xF) << 4;
  } else {  // Q6_K
    if (b < 128) {
      int h = b >> 6, k = b & 63;
      int base = h * 128 + (k & 31) + (k >= 32 ? 32 : 0);
      return (c[base] & 0xF) | (c[base + 64] & 0xF) << 4;
    }
    if (b < 192) {
      int k = b - 128, base = (k >> 5) * 128 + (k & 31);
      return (c[base] >> 4) | (c[base + 32] >> 4) << 2 | (c[base + 64] >> 4) << 4 |
             (c[base + 96] >> 4) << 6;
    }
    if (b < 208) return f.a[b - 192];
    return (f.d >> (8 * (b - 208))) & 0xFF;
  }
}

// Encode the superblocks of block ``blk`` (kWavesPerBlock waves of S
// superblocks each) of one [NB superblocks] tensor; nsb superblocks per row.
template <int TT, bool IMAT>
__device__ __forceinline__ void kq_encode_block(const float* __restrict__ x,
                                                const float* __restrict__ qw, int64_t NB,
                                                int64_t nsb, uint8_t* __restrict__ out,
                                                int64_t blk) {
  constexpr int G = Kq<TT>::G, SUBW = Kq<TT>::SUBW, BP = Kq<TT>::BP, S = 64 / G;
  __shared__ float s_sq[IMAT ? kWavesPerBlock : 1][IMAT ? S * 256 : 1];
  __shared__ uint8_t s_codes[kWavesPerBlock][S * 256];
  __shared__ SbFields s_f[kWavesPerBlock][S];
  // the make_qp_quants problems of the weighted affine types: two per superblock
  constexpr bool kQp = IMAT && (TT == CP_Q2_K || TT == CP_Q4_K || TT == CP_Q5_K);
  __shared__ QpStage<G, kQp ? 2 * kWavesPerBlock * S : 2> s_qp;

  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane % G, sl = lane / G;
  const int64_t sb0 = (blk * kWavesPerBlock + wv) * S;
  const int64_t sb = sb0 + sl;
  const bool valid = sb < NB;
  const int64_t sbr = valid ? sb : 0;  // tail lanes compute on superblock 0, write nothing

  float xv[SUBW];
  {
    const float4* p = reinterpret_cast<const float4*>(x + sbr * 256 + g * SUBW);
#pragma unroll
    for (int i = 0; i < SUBW / 4; ++i) {
      float4 v = p[i];
      xv[4 * i] = v.x;
      xv[4 * i + 1] = v.y;
      xv[4 * i + 2] = v.z;
      xv[4 * i + 3] = v.w;
    }
  }

  // importance weights qw * sqrt(k*sum(x^2)/256 + x^2)  (kquant.py:380-383, :453-455, :537-539)
  float wt[SUBW];
  if constexpr (IMAT && TT != CP_Q6_K) {
    float* sq = &s_sq[wv][sl * 256];
#pragma unroll
    for (int i = 0; i < SUBW; ++i) sq[g * SUBW + i] = xv[i] * xv[i];
    __syncthreads();
    float sx2 = sum256_lds<G>(sq, g);
    float var = (TT == CP_Q2_K ? sx2 : 2.0f * sx2) / 256.0f;
    const float4* q = reinterpret_cast<const float4*>(qw + (sbr % nsb) * 256 + g * SUBW);
#pragma unroll
    for (int i = 0; i < SUBW / 4; ++i) {
      float4 v = q[i];
      wt[4 * i] = v.x * sqrtf(var + xv[4 * i] * xv[4 * i]);
      wt[4 * i + 1] = v.y * sqrtf(var + xv[4 * i + 1] * xv[4 * i + 1]);
      wt[4 * i + 2] = v.z * sqrtf(var + xv[4 * i + 2] * xv[4 * i + 2]);
      wt[4 * i + 3] = v.w * sqrtf(var + xv[4 * i + 3] * xv[4 * i + 3]);
    }
  } else if constexpr (IMAT) {  // Q6_K: the importance vector is the weight itself
    const float4* q = reinterpret_cast<const float4*>(qw + (sbr % nsb) * 256 + g * SUBW);
#pragma unroll
    for (int i = 0; i < SUBW / 4; ++i) {
      float4 v = q[i];
      wt[4 * i] = v.x;
      wt[4 * i + 1] = v.y;
      wt[4 * i + 2] = v.z;
      wt[4 * i + 3] = v.w;
    }
  }

  int L[SUBW];
  SbFields& F = s_f[wv][sl];

  if constexpr (TT == CP_Q2_K) {
    float scale, mn;
    int sc_i, mn_i;
    float d, dmin;
    AffineFit fit;
    if constexpr (IMAT) {
      fit = fit_affine<16>(xv, wt, kQkxQ2Imat, false, true);
      float sw = psum<16>(wt);
      gfit_nonneg_pair<16>(fit.scale, fit.min, sw, 15, g, wv * S + sl, s_qp, &d, &sc_i, &dmin, &mn_i);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) wt[i] = fabsf(xv[i]);
      fit = fit_affine<16>(xv, wt, kQkxQ2Ref, true, false);
      scale = fit.scale;
      mn = fit.min;
      float smax = gmax<16>(scale), mmax = gmax<16>(mn);
      bool ps = smax > 0.0f, pm = mmax > 0.0f;
      float is = ps ? 15.0f / smax : 0.0f, im = pm ? 15.0f / mmax : 0.0f;
      sc_i = ps ? rint_magic(is * scale) : 0;
      mn_i = pm ? rint_magic(im * mn) : 0;
      d = ps ? smax / 15.0f : 0.0f;
      dmin = pm ? mmax / 15.0f : 0.0f;
    }
    uint16_t d16 = half_bits(d), m16 = half_bits(dmin);
    float dl = half_value(d16) * (float)sc_i, ml = half_value(m16) * (float)mn_i;
    if (dl != 0.0f) {
#pragma unroll
      for (int i = 0; i < 16; ++i) L[i] = clampi(rint_magic((xv[i] + ml) / dl), 0, 3);
    } else {
      affine_final_codes<16>(xv, fit, 3, L);  // the search's codes stay where dl == 0
    }
    F.a[g] = (uint8_t)((sc_i & 0xF) | (mn_i & 0xF) << 4);
    if (g == 0) {
      F.d = d16;
      F.dmin = m16;
    }
  } else if constexpr (TT == CP_Q3_K) {
    int Ls;
    float d;
    if constexpr (IMAT) {
      float scale = fit_signed<16>(xv, wt, 4, L);
      float sw = psum<16>(wt);
      d = gfit_signed<16>(scale, sw, 32, g, &Ls);
    } else {
      float scale = fit_signed_descent16(xv, 4, L);
      float amax;
      float smax = gfirst_absmax<16>(scale, g, &amax);
      bool nz = smax != 0.0f;
      float is = nz ? -32.0f / smax : 0.0f;
      Ls = nz ? clampi(rint_magic(is * scale), -32, 31) + 32 : 0;
      d = nz ? 1.0f / is : 0.0f;
      d = (nz && isfinite(d)) ? d : 0.0f;
    }
    uint16_t d16 = half_bits(d);
    float dsub = half_value(d16) * (float)(Ls - 32);
    if (dsub != 0.0f) {
#pragma unroll
      for (int i = 0; i < 16; ++i) L[i] = clampi(rint_magic(xv[i] / dsub), -4, 3) + 4;
    }
    F.a[g] = (uint8_t)Ls;
    if (g == 0) F.d = d16;
  } else if constexpr (TT == CP_Q4_K || TT == CP_Q5_K) {
    // Q5_K is Q4_K with 32 levels and its own reference-path search (kquant.py:508-593)
    constexpr int TOP = TT == CP_Q5_K ? 31 : 15;
    float scale, mn, d, dmin;
    int Ls, Lm;
    AffineFit fit;
    if constexpr (IMAT) {
      if constexpr (TT == CP_Q5_K)
        fit = fit_affine<32>(xv, wt, kQkxQ5Imat, false, true);
      else
        fit = fit_affine<32>(xv, wt, kQkxQ4Imat, false, true);
      float sw = psum<32>(wt);
      gfit_nonneg_pair<8>(fit.scale, fit.min, sw, 63, g, wv * S + sl, s_qp, &d, &Ls, &dmin, &Lm);
      if constexpr (TT == CP_Q5_K) {
        Ls = Ls < 63 ? Ls : 63;
        Lm = Lm < 63 ? Lm : 63;
      }
    } else {
      float sq[32];
#pragma unroll
      for (int i = 0; i < 32; ++i) sq[i] = xv[i] * xv[i];
      float av = sqrtf(psum<32>(sq) / 32.0f);
#pragma unroll
      for (int i = 0; i < 32; ++i) wt[i] = av + fabsf(xv[i]);
      if constexpr (TT == CP_Q5_K)
        fit = fit_affine<32>(xv, wt, kQkxQ5Ref, false, false);
      else
        fit = fit_affine<32>(xv, wt, kQkxQ4Ref, false, false);
      scale = fit.scale;
      mn = fit.min;
      float smax = gmax<8>(scale), mmax = gmax<8>(mn);
      float is = smax > 0.0f ? 63.0f / smax : 0.0f;
      float im = mmax > 0.0f ? 63.0f / mmax : 0.0f;
      // int -> uint8 narrowing wraps before the cap at 63 (kquant.py:530-532)
      Ls = (int)(uint8_t)rint_magic(is * scale);
      Lm = (int)(uint8_t)rint_magic(im * mn);
      Ls = Ls < 63 ? Ls : 63;
      Lm = Lm < 63 ? Lm : 63;
      d = smax / 63.0f;
      dmin = mmax / 63.0f;
    }
    uint16_t d16 = half_bits(d), m16 = half_bits(dmin);
    float dl = half_value(d16) * (float)Ls, ml = half_value(m16) * (float)Lm;
    if (dl != 0.0f) {
#pragma unroll
      for (int i = 0; i < 32; ++i) L[i] = clampi(rint_magic((xv[i] + ml) / dl), 0, TOP);
    } else {
      affine_final_codes<32>(xv, fit, TOP, L);  // the search's codes stay where dl == 0
    }
    F.a[g] = (uint8_t)Ls;
    F.a[8 + g] = (uint8_t)Lm;
    if (g == 0) {
      F.d = d16;
      F.dmin = m16;
    }
  } else {  // Q6_K
    if constexpr (!IMAT) {
#pragma unroll
      for (int i = 0; i < 16; ++i) wt[i] = xv[i] * xv[i];
    }
    float scale = fit_signed<16>(xv, wt, 32, L);
    float amax;
    float smax = gfirst_absmax<16>(scale, g, &amax);
    bool dead = amax < 1e-15f;
    float is = -128.0f / (dead ? 1.0f : smax);
    float d = 1.0f / is;
    int q = rint_magic(is * scale);
    int8_t sc = (int8_t)(q < 127 ? q : 127);
    uint16_t d16 = half_bits(dead ? 0.0f : d);
    float dsub = half_value(d16) * (float)sc;
    if (dsub != 0.0f && !dead) {
#pragma unroll
      for (int i = 0; i < 16; ++i) L[i] = clampi(rint_magic(xv[i] / dsub), -32, 31) + 32;
    }
    if (dead) {
#pragma unroll
      for (int i = 0; i < 16; ++i) L[i] = 0;
      sc = 0;
    }
    F.a[g] = (uint8_t)sc;
    if (g == 0) F.d = d16;
  }

  {
    uint8_t* c = &s_codes[wv][sl * 256 + g * SUBW];
#pragma unroll
    for (int i = 0; i < SUBW; i += 4) {
      uint32_t v = (uint32_t)(L[i] & 0xFF) | (uint32_t)(L[i + 1] & 0xFF) << 8 |
                   (uint32_t)(L[i + 2] & 0xFF) << 16 | (uint32_t)(L[i + 3] & 0xFF) << 24;
      *reinterpret_cast<uint32_t*>(c + i) = v;
    }
  }
  __syncthreads();

  if (sb0 >= NB) return;
  const int nvalid = (int)((NB - sb0) < S ? (NB - sb0) : S);
  const int bytes = nvalid * BP;
  uint8_t* dst = out + sb0 * BP;
  for (int dw = lane; dw < bytes / 4; dw += 64) {
    uint32_t v = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      int bi = dw * 4 + k, s = bi / BP, b = bi - s * BP;
      v |= pack_byte<TT>(&s_codes[wv][s * 256], s_f[wv][s], b) << (8 * k);
    }
    reinterpret_cast<uint32_t*>(dst)[dw] = v;
  }
  if ((bytes & 3) && lane == 0) {
    int bi = bytes - 2, s = bi / BP, b = bi - s * BP;
    uint32_t v = pack_byte<TT>(&s_codes[wv][s * 256], s_f[wv][s], b) |
                 pack_byte<TT>(&s_codes[wv][s * 256], s_f[wv][s], b + 1) << 8;
    *reinterpret_cast<uint16_t*>(dst + bi) = (uint16_t)v;
  }
}

// ---------------------------------------------------------------- decoders
// One thread per 16 consecutive weights of a superblock (16 threads per
// superblock); y = (d*sc)*q - (dmin*m) in float32 (kquant.py:416-427, :489-503,
// :596-627, :681-701).
// The 16 weights k * 16 .. k * 16 + 15 of the superblock at b (global or LDS bytes).
template <int TT>
__device__ __forceinline__ void kq_decode16(const uint8_t* __restrict__ b, int k, float (&out)[16]) {
  if constexpr (TT == CP_Q2_K) {
    float d = half_value(b[80] | b[81] << 8), dm = half_value(b[82] | b[83] << 8);
    float dl = d * (float)(b[k] & 0xF), ml = dm * (float)(b[k] >> 4);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      int e = 16 * k + i, h = e >> 7, gq = (e >> 5) & 3, l = e & 31;
      int q = (b[16 + h * 32 + l] >> (2 * gq)) & 3;
      out[i] = dl * (float)q - ml;
    }
  } else if constexpr (TT == CP_Q3_K) {
    float d = half_value(b[108] | b[109] << 8);
    const uint8_t* sc = b + 96;
    int lo = (k < 8) ? (sc[k] & 0xF) : (sc[k - 8] >> 4);
    int hi = (sc[8 + (k & 3)] >> (2 * (k >> 2))) & 3;
    float dl = d * (float)((lo | hi << 4) - 32);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      int e = 16 * k + i, h = e >> 7, gq = (e >> 5) & 3, l = e & 31;
      int q = (b[32 + h * 32 + l] >> (2 * gq)) & 3;
      int hb = (b[e & 31] >> (e >> 5)) & 1;
      out[i] = dl * (float)(q - (hb ? 0 : 4));
    }
  } else if constexpr (TT == CP_Q4_K || TT == CP_Q5_K) {
    constexpr int body = TT == CP_Q5_K ? 48 : 16;
    float d = half_value(b[0] | b[1] << 8), dm = half_value(b[2] | b[3] << 8);
    const uint8_t* sc = b + 4;
    int j = k >> 1, s, m;
    if (j < 4) {
      s = sc[j] & 63;
      m = sc[j + 4] & 63;
    } else {
      s = (sc[j + 4] & 0xF) | (sc[j - 4] >> 6) << 4;
      m = (sc[j + 4] >> 4) | (sc[j] >> 6) << 4;
    }
    float dl = d * (float)s, ml = dm * (float)m;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      int e = 16 * k + i, c = e >> 6, r = e & 63;
      int q = (r < 32) ? (b[body + c * 32 + r] & 0xF) : (b[body + c * 32 + r - 32] >> 4);
      if constexpr (TT == CP_Q5_K) q |= ((b[16 + (r & 31)] >> (2 * c + (r >> 5))) & 1) << 4;
      out[i] = dl * (float)q - ml;
    }
  } else {  // Q6_K
    float d = half_value(b[208] | b[209] << 8);
    float dl = d * (float)(int8_t)b[192 + k];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      int e = 16 * k + i, h = e >> 7, gq = (e >> 5) & 3, l = e & 31;
      int qlb = b[h * 64 + (gq & 1) * 32 + l];
      int low = (gq < 2) ? (qlb & 0xF) : (qlb >> 4);
      int high = (b[128 + h * 32 + l] >> (2 * gq)) & 3;
      out[i] = dl * (float)((low | high << 4) - 32);
    }
  }
}

// Decode 16 weights of one superblock: global thread t covers superblock t / 16.
template <int TT>
__device__ __forceinline__ void kq_decode_thread(const uint8_t* __restrict__ raw, int64_t NB,
                                                 float* __restrict__ y, int64_t t) {
  constexpr int BP = Kq<TT>::BP;
  const int64_t sb = t >> 4;
  if (sb >= NB) return;
  const int k = (int)(t & 15);
  float out[16];
  kq_decode16<TT>(raw + sb * BP, k, out);
  float4* o = reinterpret_cast<float4*>(y + sb * 256 + 16 * k);
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = make_float4(out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]);
}

// Decode of whole rows by workgroups of 4 waves, each wave 4 superblocks (1024 weights):
// the wave's container bytes arrive with dword loads (byte loads when the buffer is not
// 4-byte aligned) into LDS, every lane decodes 16 weights from there (lane = superblock
// (l / 16), 16-weight group (l % 16)), and the weights leave through LDS so that each
// store instruction writes 1 KB of consecutive floats. Waves past the end stage and store
// nothing but take part in both barriers.
constexpr int kDecSb = 4;  // superblocks per wave

template <int TT>
struct KqDecodeLds {
  static constexpr int kBytes = (kDecSb * Kq<TT>::BP + 15) / 16 * 16;
  uint8_t bytes[4][kBytes];
  float out[4][kDecSb * 256];
};

template <int TT>
__device__ __forceinline__ void kq_decode_block(const uint8_t* __restrict__ raw, int64_t NB,
                                                float* __restrict__ y, int64_t block, KqDecodeLds<TT>& L) {
  constexpr int BP = Kq<TT>::BP;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int64_t sb0 = (block * 4 + w) * kDecSb;
  const int nsb = sb0 >= NB ? 0 : (int)(NB - sb0 < kDecSb ? NB - sb0 : kDecSb);
  const int nbytes = nsb * BP;
  const uint8_t* src = raw + sb0 * BP;
  uint8_t* dst = L.bytes[w];
  if ((((uintptr_t)src) & 3) == 0) {
    const int nd = nbytes >> 2;
    for (int i = l; i < nd; i += 64)
      reinterpret_cast<uint32_t*>(dst)[i] = reinterpret_cast<const uint32_t*>(src)[i];
    for (int i = 4 * nd + l; i < nbytes; i += 64) dst[i] = src[i];
  } else {
    for (int i = l; i < nbytes; i += 64) dst[i] = src[i];
  }
  __syncthreads();
  const int s = l >> 4, k = l & 15;
  if (s < nsb) {
    float out[16];
    kq_decode16<TT>(dst + s * BP, k, out);
    float4* o = reinterpret_cast<float4*>(&L.out[w][s * 256 + 16 * k]);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = make_float4(out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]);
  }
  __syncthreads();
  const int nw = nsb * 256;
  float* yo = y + sb0 * 256;
#pragma unroll
  for (int i = 0; i < kDecSb; ++i) {
    const int idx = 256 * i + 4 * l;
    if (idx < nw) *reinterpret_cast<float4*>(yo + idx) = *reinterpret_cast<const float4*>(&L.out[w][idx]);
  }
}

// ---------------------------------------------------------------- Q8_0
// Blocks of 32 weights: d = max|x|/127 (fp16), codes int8 = round-half-away(x/d)
// (kquant.py:706-727). A wave covers 256 consecutive weights (8 blocks) with one
// float4 per lane; the 8 lanes of a block reduce max|x| with xor shuffles (max is
// exact in any order). The wave's 8*34 = 272 output bytes are assembled in LDS
// and leave as 68 dword stores.
constexpr int kQ8Bytes = 34;

// numpy's float32 -> int8 cast of sign(v)*floor(|v|+0.5) on x86: truncation to
// int32 (0x80000000 for NaN, inf and |v| >= 2^31), then the low byte. Finite
// scales keep |v| <= 127; a scale whose reciprocal overflows (max|x| < 3.7e-37)
// sends v to +-inf or NaN, and the reference then stores code 0.
__device__ __forceinline__ uint32_t q8_code(float x, float inv) {
  const float v = x * inv;
  const float a = floorf(fabsf(v) + 0.5f);
  int q = a < 2147483648.0f ? (int)a : 0;
  q = v < 0.0f ? -q : q;
  return (uint32_t)q & 0xFFu;
}

// Encode the 8 * kWavesPerBlock blocks of workgroup ``wg`` (nblk blocks in all).
// Every thread of the workgroup must call this (it holds a barrier).
__device__ __forceinline__ void q8_encode_block(const float* __restrict__ x, int64_t nblk,
                                                uint8_t* __restrict__ out, int64_t wg) {
  __shared__ uint32_t s_out[kWavesPerBlock][68];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t chunk = wg * kWavesPerBlock + wv;  // 8 blocks per chunk
  const int64_t blk = chunk * 8 + (lane >> 3);
  float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (blk < nblk) v = reinterpret_cast<const float4*>(x)[chunk * 64 + lane];
  float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  amax = fmaxf(amax, __shfl_xor(amax, 1));
  amax = fmaxf(amax, __shfl_xor(amax, 2));
  amax = fmaxf(amax, __shfl_xor(amax, 4));
  const float d = amax / 127.0f;
  const float inv = d != 0.0f ? 1.0f / d : 0.0f;
  const uint32_t codes = q8_code(v.x, inv) | q8_code(v.y, inv) << 8 | q8_code(v.z, inv) << 16 |
                         q8_code(v.w, inv) << 24;
  uint16_t* so = reinterpret_cast<uint16_t*>(s_out[wv]);
  const int h = (lane >> 3) * (kQ8Bytes / 2) + 1 + 2 * (lane & 7);  // in halfwords
  so[h] = (uint16_t)codes;
  so[h + 1] = (uint16_t)(codes >> 16);
  if ((lane & 7) == 0) so[h - 1] = half_bits(d);
  __syncthreads();
  if (chunk * 8 >= nblk) return;
  const int64_t nvalid = nblk - chunk * 8 < 8 ? nblk - chunk * 8 : 8;
  const int bytes = (int)nvalid * kQ8Bytes;
  uint8_t* dst = out + chunk * 8 * kQ8Bytes;
  for (int dw = lane; dw < bytes / 4; dw += 64) reinterpret_cast<uint32_t*>(dst)[dw] = s_out[wv][dw];
  if ((bytes & 3) && lane == 0)
    reinterpret_cast<uint16_t*>(dst)[bytes / 2 - 1] = so[bytes / 2 - 1];
}

// Decode 4 consecutive weights (global thread t): y = d * code in float32.
__device__ __forceinline__ void q8_decode_thread(const uint8_t* __restrict__ raw, int64_t nblk,
                                                 float* __restrict__ y, int64_t t) {
  const int64_t blk = t >> 3;
  if (blk >= nblk) return;
  const uint16_t* b = reinterpret_cast<const uint16_t*>(raw + blk * kQ8Bytes);
  const int j = (int)(t & 7);
  const float d = half_value(b[0]);
  const uint32_t c = (uint32_t)b[1 + 2 * j] | (uint32_t)b[2 + 2 * j] << 16;
  reinterpret_cast<float4*>(y)[t] =
      make_float4(d * (float)(int8_t)(c & 0xFF), d * (float)(int8_t)((c >> 8) & 0xFF),
                  d * (float)(int8_t)((c >> 16) & 0xFF), d * (float)(int8_t)(c >> 24));
}

}  // namespace cp
