// Wave-pipeline fused causal long convolution for two-stage plans (N = R0*R1 = 2L).
//
// One 64-lane wavefront carries one pair of sequences of one channel -- packed as
// the real and imaginary parts of a single complex transform -- through every
// stage of the forward transform, the spectrum product and the inverse transform
// in VGPRs: no LDS exchange and no barrier between stages. Only the pair's input
// and output pass through a per-wavefront LDS scratch, so that global memory is
// read and written in whole rows.
//
// Why it works (v_mfma_f32_16x16x32_f16, complex K interleave of fftconv.hpp):
// a result tile D[i][j] sits in lane (j, g) as rows i = 4g..4g+3; an operand
// fragment of the next contraction over i wants lane (j, g) to hold K indices
// 4g..4g+3 for row/column j. They coincide, so each stage's accumulator tile,
// twiddled and rounded to fp16, IS the next stage's operand with the roles of the
// two indices swapped:
//   phase 1  D1[m][k0]  = sum_{n0<R0/2} x[n0*M+m] F0[n0][k0]       (A = data, B = F0)
//            B2[m][k0]  = fp16(D1 * sc0 * w^(m k0))                 -> B operand over m
//   phase 2  D2[k1][k0] = sum_m F1[k1][m] B2[m][k0]                 (A = F1)
//            A2[k0][k1] = fp16(conj(D2 * Kf))                       -> A operand over k1
//            E[k0][n1]  = sum_k1 A2[k0][k1] F1[k1][n1]              (B = F1)
//            A3[n1][k0] = fp16(E * sc1 * sc0 * w^(k0 n1))           -> A operand over k0
//   phase 3  y_a[n0*M+m] =  Re sum_k0 A3[m][k0] F0[k0][n0],  y_b = -Im (n0 < R0/2)
// which is the reference's schedule L0f -> Rf(x Kf) -> Ri -> L0i (src/sffft.cu:273-279)
// with its digit order (src/sffft.cu:106-113, 283-288) and fp16 storage between
// stages (src/sffft.cu:120-135); the inverse is computed as conj(DFT(conj X)).
//
// Read-only tables in LDS, filled once per workgroup:
//   F0, F1 : DFT fragments of radix R0 and R1, both kinds ([cos | sin] and
//            [-sin | cos]) in the order of the coefficient table (the first kind
//            only when both do not fit beside the spectra, see WavePlan)
//   TW1    : sc0 * w^(m k0) in the lane order of the phase-1 result tiles
//   TW2    : sc1 * sc0 * w^(k0 n1) in the lane order of the inverse result tiles
// so no twiddle is evaluated in the loop and no per-stage scale is applied; the
// output scale 1/sqrt(R0) rides on TW2 and 1/sqrt(R1) on the spectrum. With
// R0 == R1 the two tables hold the same function of the same tile and lane
// indices, so TW2 is TW1 and the spectrum carries sc1 as well (1/R1).
// The channel spectra sit in LDS when they fit beside the tables and the operand
// scratch; otherwise the wavefronts read them from global memory (L2-resident:
// B/2 wavefronts read each channel's spectrum). A real filter's spectrum is
// Hermitian, K[N-k] = conj(K[k]), so only its columns k0 = 0..R0/2 are stored (about
// half the bytes, WavePlan::hs_index) and the lanes of columns k0 > R0/2 read the
// partner frequency N-k and conjugate it; complex filters (HERM = false) read the
// whole spectrum.
//
// fp16 products (HP: the fp16-accumulation mode, real filters): the two twiddle tables
// hold fp16 values, [wr0..wr3 | wi0..wi3] per lane and tile (one 16-byte read instead of
// two), and the twiddle products run in packed fp16 on the accumulators rounded to fp16
// (v_cvt_pk_f16_f32, v_pk_mul_f16, v_pk_fma_f16: 12 VALU instructions per tile instead of
// 16, the mode's accumulator rounding included). Each product then carries about three
// fp16 roundings instead of one: the speed-for-precision trade of the reference's fp16
// accumulation (README.md:112-122). fp32 accumulation keeps fp32 twiddles and products.
#pragma once
#include "fftconv.hpp"

// k0 strips per phase-2 step when the DFT fragments are read from LDS (not held)
#ifndef SFFFT_WAVE_STRIPS
#define SFFFT_WAVE_STRIPS 2
#endif

namespace sffft {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int R0_, int R1_>
struct WavePlan {
  static constexpr int R0 = R0_, R1 = R1_, N = R0 * R1, L = N / 2, M = R1;
  static constexpr int MT = R1 / 16;                  // 16-wide tiles of m = n1 (and of k1)
  static constexpr int ST = R0 / 16;                  // 16-wide strips of k0
  static constexpr int KS1 = R0 >= 32 ? R0 / 32 : 1;  // phase-1 K steps (n0 < R0/2 only)
  static constexpr int NT3 = R0 >= 32 ? R0 / 32 : 1;  // phase-3 result tiles (n0 < R0/2 only)
  static constexpr int F0_H8 = ST * ST * 128;  // both fragment kinds
  static constexpr int F1_H8 = R1 == R0 ? 0 : MT * MT * 128;
  static constexpr int TW_F4 = N / 2;  // one twiddle table: N complex fp32 = N/2 float4
  // one twiddle table in the table format of the kernel: fp32, or with fp16 products (hp)
  // N complex fp16 = N/4 float4
  static constexpr int twb_f4(bool hp) { return hp ? N / 4 : N / 2; }
  static constexpr int SP_F4 = N / 2;  // one channel's whole spectrum: N complex64 = N/2 float4
  // One channel's Hermitian half spectrum (hs_index): columns k0 = 0..R0/2 of HPITCH
  // float4 each (8*MT values and one of padding: an odd pitch puts the 16 columns a
  // lane group reads on 16 distinct 16-byte slots).
  static constexpr int HPITCH = 8 * MT + 1;
  static constexpr int HSP_F4 = (R0 / 2 + 1) * HPITCH;
  static constexpr int sp_f4(bool herm) { return herm ? HSP_F4 : SP_F4; }
  // ch channels' spectra in LDS, in whole 64-float4 runs of the table copy
  static constexpr int spl_f4(int ch, bool herm) { return (ch * sp_f4(herm) + 63) / 64 * 64; }
  static constexpr int TW_TABLES = R0 == R1 ? 1 : 2;
  static constexpr int tab_f4(bool hp) { return F0_H8 + F1_H8 + TW_TABLES * twb_f4(hp); }
  // the same with the first fragment kind only (the second is derived in registers)
  static constexpr int tab1_f4(bool hp) { return (F0_H8 + F1_H8) / 2 + TW_TABLES * twb_f4(hp); }
  // per-wavefront operand scratch of the row loads with fp32 I/O (bf16 needs less)
  static constexpr int SCRATCH_MAX = 16 * (M + 4) * 4;
  // Layout for a workgroup of nw wavefronts serving ch channels, in order of preference:
  // both DFT fragment kinds and the spectra in LDS; the first kind only with the spectra
  // in LDS; the first kind only with the spectra read through L2. Every layout reads the
  // pairs as row chunks through the operand scratch.
  // hp: the fp16 twiddle tables of the fp16-products kernels (half the bytes).
  static constexpr bool both_kinds(int ch, int nw, bool herm = true, bool hp = false) {
    return (tab_f4(hp) + spl_f4(ch, herm)) * 16 + nw * SCRATCH_MAX <= 163840;
  }
  static constexpr int tables_f4(int ch, int nw, bool herm = true, bool hp = false) {
    return both_kinds(ch, nw, herm, hp) ? tab_f4(hp) : tab1_f4(hp);
  }
  static constexpr bool spectra_in_lds(int ch, int nw, bool herm = true, bool hp = false) {
    return (tables_f4(ch, nw, herm, hp) + spl_f4(ch, herm)) * 16 + nw * SCRATCH_MAX <= 163840;
  }
  static constexpr int lds_bytes(int ch, int nw, bool herm = true, bool hp = false) {
    return (tables_f4(ch, nw, herm, hp) + (spectra_in_lds(ch, nw, herm, hp) ? spl_f4(ch, herm) : 0)) * 16 +
           nw * SCRATCH_MAX;
  }
  static_assert(R0 >= 16 && R0 <= 64 && R1 >= 16 && R1 <= 64, "radices are 16, 32 or 64");
};

// Twiddle-table index of lane `lane`, tile (a, b), float4 q (q = 0: values 0,1; q = 1: 2,3).
// Split layout: each float4 of a tile in its own run of 64 lanes, so that the lanes of one
// 16-byte read are 16 bytes apart and fall on distinct banks. Paired layout: both float4 of
// a lane side by side; lanes are 32 bytes apart, and lanes l and l+4 of every 8-lane pass
// share banks (two-way conflicts on every twiddle read, all of the kernel's conflicts). The
// paired layout is kept for 64x64, whose 168-VGPR kernel spills with the split one (its
// two reads per tile then need two lane offsets): 5% slower there, 3% faster at 64x32.
__host__ __device__ constexpr bool tw_split(int r0, int r1) { return !(r0 == 64 && r1 == 64); }
__host__ __device__ constexpr int tw_index(bool split, int tile, int lane, int q) {
  return split ? (tile * 2 + q) * 64 + lane : (tile * 64 + lane) * 2 + q;
}
// Spectrum index (float4 units) in the wave pipeline's order: tile = s*MT + kt,
// q as above; lanes at 16-byte stride so one load instruction reads 1 KB.
__host__ __device__ constexpr int sp_index(int tile, int lane, int q) { return (tile * 2 + q) * 64 + lane; }
// Hermitian half spectrum (float4 units): the float4 at hs_index(k0, kt, q, g) holds the
// values k1 = 16kt + 4g + 2q and +1 of column k0 <= R0/2, i.e. K[k0 + R0*k1]. Column
// R0/2 is stored in the form its own lanes read it as a partner (see herm_spectrum_pack):
// conj(K[R0/2 + R0*(R1 - 1 - k1)]) at k1.
template <class P>
__host__ __device__ constexpr int hs_index(int k0, int kt, int q, int g) {
  return k0 * P::HPITCH + (kt * 2 + q) * 4 + g;
}

// DFT fragment (a, b, kind) of a radix-R table in LDS: coefficient-table order, or
// with K1 the first kind [cos | sin] only. The second kind [-sin | cos] is then the
// first with its halves swapped and the new first half negated: read with the halves
// exchanged, then two sign flips. This is exact, as the table rounds -sin to the
// negation of the rounded sin.
template <int R, bool K1 = false>
__device__ __forceinline__ h8 dft_frag(const h8* F, int a, int b, int kind, int lane) {
  if constexpr (K1) {
    const u32x2* p = reinterpret_cast<const u32x2*>(F + (a * (R / 16) + b) * 64 + lane);
    const u32x2 c = p[0], s = p[1];
    if (kind == 0) return __builtin_bit_cast(h8, (u32x4){c.x, c.y, s.x, s.y});
    return __builtin_bit_cast(h8, (u32x4){s.x ^ 0x80008000u, s.y ^ 0x80008000u, c.x, c.y});
  } else {
    return F[((a * (R / 16) + b) * 2 + kind) * 64 + lane];
  }
}

// (dr + i di) * w for four values, packed as an operand fragment [re | im] in fp16.
__device__ __forceinline__ h8 cmul_pack(f4 dr, f4 di, float4 w01, float4 w23) {
  const float wr[4] = {w01.x, w01.z, w23.x, w23.z};
  const float wi[4] = {w01.y, w01.w, w23.y, w23.w};
  h8 o;
#pragma unroll
  for (int v = 0; v < 4; v++) {
    o[v] = (_Float16)(dr[v] * wr[v] - di[v] * wi[v]);
    o[4 + v] = (_Float16)(dr[v] * wi[v] + di[v] * wr[v]);
  }
  return o;
}

// The same as a product in packed fp16 (the fp16-accumulation mode, cmul_hp): the
// accumulators rounded to fp16, w from the fp16 table as [wr0 wr1 wr2 wr3 | wi0 wi1 wi2 wi3].
__device__ __forceinline__ h8 cmul_pack_h(f4 dr, f4 di, h8 w) {
  const HW hw{(h2){w[0], w[1]}, (h2){w[2], w[3]}, (h2){w[4], w[5]}, (h2){w[6], w[7]}};
  h4 xr, xi;
  cmul_hp(dr, di, hw, xr, xi);
  return join_h8(xr, xi);
}

// conj((dr + i di) * k) for four spectrum values k (float4 pairs of complex64); with
// CONJ the values given are conj(k) (the signs of the products absorb the conjugation).
template <bool CONJ = false>
__device__ __forceinline__ h8 spectrum_conj_pack(f4 dr, f4 di, float4 k01, float4 k23) {
  const float kr[4] = {k01.x, k01.z, k23.x, k23.z};
  const float ki[4] = {k01.y, k01.w, k23.y, k23.w};
  h8 o;
#pragma unroll
  for (int v = 0; v < 4; v++) {
    if constexpr (CONJ) {
      o[v] = (_Float16)(dr[v] * kr[v] + di[v] * ki[v]);
      o[4 + v] = (_Float16)(dr[v] * ki[v] - di[v] * kr[v]);
    } else {
      o[v] = (_Float16)(dr[v] * kr[v] - di[v] * ki[v]);
      o[4 + v] = (_Float16)(-(dr[v] * ki[v] + di[v] * kr[v]));
    }
  }
  return o;
}

// spectrum_conj_pack, or with HP (the fp16-accumulation mode) the same product in packed
// fp16 on the raw accumulators (cmul_hp, conjugated)
template <bool CONJ, bool HP>
__device__ __forceinline__ h8 spec_pack(f4 dr, f4 di, float4 k01, float4 k23) {
  if constexpr (HP) {
    const float kr[4] = {k01.x, k01.z, k23.x, k23.z};
    const float ki[4] = {CONJ ? -k01.y : k01.y, CONJ ? -k01.w : k01.w, CONJ ? -k23.y : k23.y, CONJ ? -k23.w : k23.w};
    h4 xr, xi;
    cmul_hp<true>(dr, di, hw_of(kr, ki), xr, xi);
    return join_h8(xr, xi);
  } else {
    return spectrum_conj_pack<CONJ>(dr, di, k01, k23);
  }
}

// conj(D * K) for lane (j, g) of the phase-2 tile of strip s and k1 tile kt, from a
// Hermitian half spectrum: K at k0 = 16s + j and k1 = 16kt + 4g + v, v = 0..3. Columns
// k0 < R0/2 are read directly. A column k0 >= R0/2 holds conj(K) of the partner
// frequency N - k: column R0 - k0 and k1' = R1 - 1 - k1, so the lane reads tile
// MT-1-kt, lane group 3-g and the other float4 of its pair, in reverse value order.
// For R0 >= 32 a strip is wholly direct or wholly partner (no per-lane choice); with
// R0 = 16 the single strip splits at lane j = 8.
template <class P, bool HP = false>
__device__ __forceinline__ h8 herm_spectrum_pack(f4 dr, f4 di, const float4* SP, int s, int kt, int lane) {
  constexpr int R0 = P::R0, MT = P::MT;
  const int j = lane & 15, g = lane >> 4;
  const int dk0 = 16 * s + j, pk0 = R0 - 16 * s - j;
  if (16 * s + 15 < R0 / 2) {
    return spec_pack<false, HP>(dr, di, SP[hs_index<P>(dk0, kt, 0, g)], SP[hs_index<P>(dk0, kt, 1, g)]);
  } else if (16 * s >= R0 / 2) {
    // p0: conj(K) of v = 1, 0; p1: of v = 3, 2
    const float4 p0 = SP[hs_index<P>(pk0, MT - 1 - kt, 1, 3 - g)];
    const float4 p1 = SP[hs_index<P>(pk0, MT - 1 - kt, 0, 3 - g)];
    return spec_pack<true, HP>(dr, di, make_float4(p0.z, p0.w, p0.x, p0.y), make_float4(p1.z, p1.w, p1.x, p1.y));
  } else {
    const bool dir = dk0 < R0 / 2;
    const float4 a0 = SP[dir ? hs_index<P>(dk0, kt, 0, g) : hs_index<P>(pk0, MT - 1 - kt, 1, 3 - g)];
    const float4 a1 = SP[dir ? hs_index<P>(dk0, kt, 1, g) : hs_index<P>(pk0, MT - 1 - kt, 0, 3 - g)];
    const float4 k01 = dir ? a0 : make_float4(a0.z, -a0.w, a0.x, -a0.y);
    const float4 k23 = dir ? a1 : make_float4(a1.z, -a1.w, a1.x, -a1.y);
    return spec_pack<false, HP>(dr, di, k01, k23);
  }
}

template <bool ACC16>
__device__ __forceinline__ f4 acc_round(f4 v) {
  if constexpr (ACC16) {
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = (float)(_Float16)v[i];
  }
  return v;
}

__device__ __forceinline__ float4 ld_f4(const float4* p) { return *p; }


// 16-byte blocks copied from global memory straight into LDS (global_load_lds_dwordx4:
// lane i of the wave writes bytes [16i, 16i+16) after the wave-uniform LDS base).
// COUNT blocks in runs of 64, run r by wave r mod NW. Every wave issues exactly
// dma_issues<COUNT, NW>() instructions (a wave without a run of its own in the last
// round copies the last run again: same source, same bytes, same place), so the
// caller knows how many vector-memory operations follow.
template <int COUNT, int NW>
__host__ __device__ constexpr int dma_issues() { return (COUNT / 64 + NW - 1) / NW; }

template <int COUNT, int NW, class SRC>
__device__ __forceinline__ void dma_to_lds(float4* dst, SRC src, int lane, int wave) {
  static_assert(COUNT % 64 == 0, "tables are whole 64-block runs");
  constexpr int RUNS = COUNT / 64;
#pragma unroll
  for (int i = 0; i < dma_issues<COUNT, NW>(); i++) {
    int run = i * NW + wave;
    if (RUNS % NW != 0 && run >= RUNS) run = RUNS - 1;
    __builtin_amdgcn_global_load_lds(src(run * 64 + lane), (__attribute__((address_space(3))) void*)(dst + run * 64),
                                     16, 0, 0);
  }
}

// s_waitcnt with the given vector-memory count and no wait on the other counters
// (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
// The count saturates at 63: with more operations in flight, waiting for 63 still
// completes everything issued before the last 63 (the counter retires in order).
template <int VM>
__device__ __forceinline__ void wait_vmcnt() {
  constexpr int V = VM > 63 ? 63 : VM;
  static_assert(VM >= 0, "vmcnt is not negative");
  __builtin_amdgcn_s_waitcnt((V & 15) | ((V >> 4) << 14) | (7 << 4) | (15 << 8));
}

// DFT fragments of radix R (both kinds, or with K1 the first only) computed into LDS
// (the in-kernel "legacy" source), in coefficient-table order.
template <int R, int NTH, bool K1 = false>
__device__ __forceinline__ void compute_dft(h8* dst, int tid) {
  constexpr int T = R / 16, KINDS = K1 ? 1 : 2, TOTAL = T * T * 64 * KINDS;
#pragma unroll
  for (int i = 0; i < (TOTAL + NTH - 1) / NTH; i++) {
    const int k = tid + i * NTH;
    if (TOTAL % NTH == 0 || k < TOTAL) {
      const int ab = k / (64 * KINDS), kind = K1 ? 0 : (k >> 6) & 1;
      dst[k] = cf_frag<R, false>(nullptr, ab / T, ab % T, kind, k & 63);
    }
  }
}

// Global loads of one pair. The first L samples of a row are the non-zero half of
// its length-2L transform input and are contiguous, so both rows are read as 16-byte
// chunks, one KB per instruction, with the streaming (non-temporal) hint: chunk q of
// the pair (rows a then b) goes to lane q % 64 of round q / 64.

template <class P, class TIO>
struct PairLoads {
  static constexpr int EPC = 16 / (int)sizeof(TIO);  // samples per chunk
  static constexpr int CPS = P::L / EPC;              // chunks per row
  static constexpr int ROUNDS = (2 * CPS + 63) / 64;  // load instructions per pair
  u32x4 c[ROUNDS];
};

// Vector-memory instructions issue_pair_loads emits.
template <class P, class TIO>
__host__ __device__ constexpr int pair_load_issues() { return PairLoads<P, TIO>::ROUNDS; }

template <class P, class TIO>
__device__ __forceinline__ void issue_pair_loads(const TIO* __restrict__ xa, const TIO* __restrict__ xb,
                                                 PairLoads<P, TIO>& d, int lane) {
  typedef PairLoads<P, TIO> D;
#pragma unroll
  for (int i = 0; i < D::ROUNDS; i++) {
    const int q = i * 64 + lane;
    if (2 * D::CPS >= (i + 1) * 64 || q < 2 * D::CPS) {
      const TIO* row = q < D::CPS ? xa : xb;
      const int off = q < D::CPS ? q : q - D::CPS;
      d.c[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row) + off);
    }
  }
}

// Per-wavefront LDS scratch that turns the row chunks into phase-1 operands: 16 rows
// (one K step of n0) of M samples at a pitch chosen so that the four K groups of a
// wavefront read four disjoint 16-bank ranges and every row start stays 16-byte aligned.
template <class P, class TIO>
__host__ __device__ constexpr int scratch_pitch() { return P::M + (sizeof(TIO) == 4 ? 4 : 8); }
template <class P, class TIO>
__host__ __device__ constexpr int scratch_bytes() { return 16 * scratch_pitch<P, TIO>() * (int)sizeof(TIO); }

__device__ __forceinline__ float io_to_f32_lds(const float* p) { return *p; }
__device__ __forceinline__ float io_to_f32_lds(const uint16_t* p) { return __uint_as_float((uint32_t)*p << 16); }

// Phase-1 A operands a[mt][ks] (slots 0..3 row a, 4..7 row b; n0 = 16ks + 4g + j,
// m = 16mt + r) from the pair's chunks, through the wave's scratch S. With SPLIT each
// fp32 sample x enters as fp16(x) in a and its remainder fp16(x - fp16(x)) in alo, so
// that phase 1 sees x to about 22 bits instead of 11.
template <class P, class TIO, bool SPLIT>
__device__ __forceinline__ void pair_operands(const PairLoads<P, TIO>& d, TIO* S, h8 (*a)[P::KS1],
                                              h8 (*alo)[P::KS1], int lane) {
  typedef PairLoads<P, TIO> D;
  constexpr int R0 = P::R0, M = P::M, PITCH = scratch_pitch<P, TIO>();
  constexpr int ROWS = R0 / 2 < 16 ? R0 / 2 : 16;  // non-zero rows per K step
  const int r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int ks = 0; ks < P::KS1; ks++)
#pragma unroll
    for (int sq = 0; sq < 2; sq++) {
      // chunks of rows [16ks, 16ks + ROWS) of row sq
      constexpr int PER = ROWS * M / D::EPC;
      const int lo = sq * D::CPS + ks * (16 * M / D::EPC);
#pragma unroll
      for (int i = 0; i < D::ROUNDS; i++) {
        const int q = i * 64 + lane;
        if (q >= lo && q < lo + PER) {
          const int e = (q - lo) * D::EPC;
          *reinterpret_cast<u32x4*>(S + (e / M) * PITCH + e % M) = d.c[i];
        }
      }
      // A lane reads what other lanes wrote: without the fences a lane that wrote
      // nothing here would reuse its reads of the previous block, and writes could be
      // moved above the previous block's reads.
      wave_lds_fence();
#pragma unroll
      for (int mt = 0; mt < P::MT; mt++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const bool live = 4 * g + j < ROWS;
          const float v = live ? io_to_f32_lds(S + (4 * g + j) * PITCH + 16 * mt + r) : 0.f;
          const _Float16 hi = (_Float16)v;
          a[mt][ks][4 * sq + j] = hi;
          if constexpr (SPLIT) alo[mt][ks][4 * sq + j] = (_Float16)(v - (float)hi);
        }
      wave_lds_fence();
    }
}

// Output of one 16-row block (rows n0 = 16nu + c of the MT result tiles; lane (c, g)
// holds m = 16t + 4g .. +3 of tile t) of one sequence, through the wave's scratch S,
// so that every store instruction writes whole rows: lane q of round i stores
// 16-byte chunk q % CPR of row q / CPR (for fp32 rows of 32 samples, 8 rows of 128
// bytes, one KB contiguous). Whole lines allow the streaming (non-temporal) hint:
// each line is written once, and held dirty in the XCD's L2 it would be written back
// by the end-of-kernel release after the last wave instead of during the run
// (streaming stores of partial lines would reach HBM as partial writes).
// Rows from ROWS3 on (the zero half of R0 = 16) are not stored.
__device__ __forceinline__ void put4(float* p, f4 v) { *reinterpret_cast<f4*>(p) = v; }
__device__ __forceinline__ void put4(uint16_t* p, f4 v) { *reinterpret_cast<u32x2*>(p) = f4_to_bf16x4(v); }

template <class P, class TIO>
__device__ __forceinline__ void store_rows(TIO* S, const f4 (&z)[P::MT], TIO* __restrict__ y, int lane) {
  constexpr int M = P::M, PITCH = scratch_pitch<P, TIO>(), EPC = 16 / (int)sizeof(TIO), CPR = M / EPC;
  constexpr int ROWS3 = P::R0 >= 32 ? 16 : P::R0 / 2, ROUNDS = (16 * CPR + 63) / 64;
  const int c = lane & 15, g = lane >> 4;
#pragma unroll
  for (int t = 0; t < P::MT; t++) put4(S + c * PITCH + 16 * t + 4 * g, z[t]);
  // other lanes' writes are read below
  wave_lds_fence();
#pragma unroll
  for (int i = 0; i < ROUNDS; i++) {
    const int q = i * 64 + lane, row = q / CPR, col = (q % CPR) * EPC;
    if (row < ROWS3)
      __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(S + row * PITCH + col),
                                  reinterpret_cast<u32x4*>(y + row * M + col));
  }
  wave_lds_fence();
}

// Every stage of one pair, from its loaded operands to the stored outputs; SP is the
// channel's spectrum in LDS. SPLIT: fp32 input as value plus remainder (pair_operands),
// two MFMAs per phase-1 product into the same accumulator.
template <class P, class TIO, bool ACC16, bool HOLD_F1, bool K1, bool HERM, bool SPLIT, bool HP>
__device__ __forceinline__ void process_pair(const PairLoads<P, TIO>& d, TIO* S, const float4* SP,
                                             TIO* __restrict__ ya, TIO* __restrict__ yb, const h8* F0,
                                             const h8* F1, const float4* TW1, const float4* TW2, int lane) {
  constexpr int R0 = P::R0, M = P::M, MT = P::MT, ST = P::ST, KS1 = P::KS1, NT3 = P::NT3;
  constexpr bool TWS = tw_split(P::R0, P::R1);  // twiddle-table layout (tw_index)
  // twiddled tile t of the table TW: fp32 table and products, or (HP) fp16 table and
  // packed fp16 products, whose conversion to fp16 is the accumulator's rounding
  auto twiddled = [&](const float4* TW, int t, f4 dr, f4 di) -> h8 {
    if constexpr (HP) {
      return cmul_pack_h(dr, di, reinterpret_cast<const h8*>(TW)[t * 64 + lane]);
    } else {
      return cmul_pack(acc_round<ACC16>(dr), acc_round<ACC16>(di), TW[tw_index(TWS, t, lane, 0)],
                       TW[tw_index(TWS, t, lane, 1)]);
    }
  };
  // With 16 tiles per transform (64x64) the pair alone fills 64 VGPRs; compiler-only
  // barriers at the top of each tile step keep the next step's table and spectrum
  // loads from being hoisted over the current one, which would not fit beside it.
  constexpr bool LEAN = MT * ST >= 16;
  auto step_fence = [] {
    if constexpr (LEAN) __asm__ volatile("" ::: "memory");
  };

  // ---- phase 1: DFT over n0 (first R0/2 rows only), twiddle, -> B2[m tile][k0 strip]
  h8 a[MT][KS1], alo[SPLIT ? MT : 1][KS1];
  pair_operands<P, TIO, SPLIT>(d, S, a, alo, lane);
  h8 b2[MT][ST];
#pragma unroll
  for (int nt = 0; nt < ST; nt++) {
    step_fence();
    h8 f0[KS1], f1[KS1];
#pragma unroll
    for (int ks = 0; ks < KS1; ks++) {
      f0[ks] = dft_frag<R0, K1>(F0, nt, ks, 0, lane);
      f1[ks] = dft_frag<R0, K1>(F0, nt, ks, 1, lane);
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
      f4 dr = {0.f, 0.f, 0.f, 0.f}, di = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS1; ks++) {
        dr = mfma(a[mt][ks], f0[ks], dr);
        di = mfma(a[mt][ks], f1[ks], di);
        if constexpr (SPLIT) {
          dr = mfma(alo[mt][ks], f0[ks], dr);
          di = mfma(alo[mt][ks], f1[ks], di);
        }
      }
      b2[mt][nt] = twiddled(TW1, mt * ST + nt, dr, di);
    }
  }

  // ---- phase 2: per k0 strip, DFT over n1, spectrum, inverse DFT over k1, twiddle
  h8 g0[HOLD_F1 ? MT : 1][HOLD_F1 ? MT : 1][2];
  if constexpr (HOLD_F1) {
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
      for (int k = 0; k < MT; k++)
#pragma unroll
        for (int kind = 0; kind < 2; kind++) g0[i][k][kind] = dft_frag<P::R1, K1>(F1, i, k, kind, lane);
  }
  auto f1frag = [&](int i, int k, int kind) -> h8 {
    if constexpr (HOLD_F1) return g0[i][k][kind];
    else return dft_frag<P::R1, K1>(F1, i, k, kind, lane);
  };
  // Strips are taken SG at a time, so that each DFT fragment read from LDS (and, with
  // the first kind only, each second kind rebuilt from it) serves SG strips: without
  // held fragments phase 2 is bound by these LDS reads. The accumulation order of every
  // output is the same for any SG.
  constexpr int SG = HOLD_F1 ? 1 : SFFFT_WAVE_STRIPS;
  static_assert(ST % SG == 0, "whole strip groups");
#pragma unroll
  for (int s0 = 0; s0 < ST; s0 += SG) {
    h8 a2[SG][MT];
#pragma unroll
    for (int kt = 0; kt < MT; kt++) {
      step_fence();
      f4 dr[SG], di[SG];
#pragma unroll
      for (int j = 0; j < SG; j++) dr[j] = di[j] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int mt = 0; mt < MT; mt++) {
        const h8 fa = f1frag(kt, mt, 0), fb = f1frag(kt, mt, 1);
#pragma unroll
        for (int j = 0; j < SG; j++) {
          dr[j] = mfma(fa, b2[mt][s0 + j], dr[j]);
          di[j] = mfma(fb, b2[mt][s0 + j], di[j]);
        }
      }
#pragma unroll
      for (int j = 0; j < SG; j++) {
        const int s = s0 + j, tile = s * MT + kt;
        // HP rounds the raw accumulators itself
        const f4 r = HP ? dr[j] : acc_round<ACC16>(dr[j]), i = HP ? di[j] : acc_round<ACC16>(di[j]);
        if constexpr (HERM)
          a2[j][kt] = herm_spectrum_pack<P, HP>(r, i, SP, s, kt, lane);
        else
          a2[j][kt] = spectrum_conj_pack(r, i, SP[sp_index(tile, lane, 0)], SP[sp_index(tile, lane, 1)]);
      }
    }
#pragma unroll
    for (int t = 0; t < MT; t++) {
      step_fence();
      f4 er[SG], ei[SG];
#pragma unroll
      for (int j = 0; j < SG; j++) er[j] = ei[j] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kt = 0; kt < MT; kt++) {
        const h8 fa = f1frag(t, kt, 0), fb = f1frag(t, kt, 1);
#pragma unroll
        for (int j = 0; j < SG; j++) {
          er[j] = mfma(a2[j][kt], fa, er[j]);
          ei[j] = mfma(a2[j][kt], fb, ei[j]);
        }
      }
#pragma unroll
      for (int j = 0; j < SG; j++) {
        b2[t][s0 + j] = twiddled(TW2, (s0 + j) * MT + t, er[j], ei[j]);
      }
    }
  }

  // ---- phase 3: inverse DFT over k0 for n0 < R0/2; real part -> row a, -imag -> row b
#pragma unroll
  for (int nu = 0; nu < NT3; nu++) {
    step_fence();
    h8 f0[ST], f1[ST];
#pragma unroll
    for (int s = 0; s < ST; s++) {
      f0[s] = dft_frag<R0, K1>(F0, nu, s, 0, lane);
      f1[s] = dft_frag<R0, K1>(F0, nu, s, 1, lane);
    }
    f4 za[MT] = {}, zb[MT] = {};
#pragma unroll
    for (int t = 0; t < MT; t++) {
#pragma unroll
      for (int s = 0; s < ST; s++) {
        za[t] = mfma(b2[t][s], f0[s], za[t]);
        zb[t] = mfma(b2[t][s], f1[s], zb[t]);
      }
      za[t] = acc_round<ACC16>(za[t]);
      zb[t] = -acc_round<ACC16>(zb[t]);  // row b is minus the imaginary part
    }
    store_rows<P, TIO>(S, za, ya + 16 * nu * M, lane);
    store_rows<P, TIO>(S, zb, yb + 16 * nu * M, lane);
  }
}

// grid = ceil(H / CH) workgroups of 64*NW lanes. Workgroup w takes channels
// [w*CH, w*CH + CH) and their CH*(B/2) pairs, pair p = c*(B/2) + bp: rows (2bp, h)
// and (2bp+1, h), h = w*CH + c. Wave v takes pairs v, v + NW, ... The DFT and
// twiddle tables and the CH channel spectra are copied into LDS once, so the
// B/2 wavefronts of a channel read its spectrum from LDS rather than each from L2.
// HERM: kf holds Hermitian half spectra (real filters, hs_index, HSP_F4 float4 at the
// start of each channel's row); otherwise whole spectra (complex filters, sp_index, SP_F4
// per channel). The rows of kf are SP_F4 float4 (2L complex64) apart in both cases.
template <class P, int NW, int CH, class TIO, bool CACHED, bool ACC16, bool HERM>
__global__ void __launch_bounds__(64 * NW)
    fftconv_wave_kernel(const TIO* __restrict__ u, const float4* __restrict__ kf, TIO* __restrict__ y, int B,
                        int H, const h8* __restrict__ ftab, const float4* __restrict__ twtab) {
  constexpr int R0 = P::R0;
  // fp16 products: the fp16-accumulation mode (real filters)
  constexpr bool HP = HERM && ACC16;
#ifdef SFFFT_WAVE_FORCE_K1
  constexpr bool K1 = true;
#else
  constexpr bool K1 = !P::both_kinds(CH, NW, HERM, HP);  // first DFT fragment kind only
#endif
  constexpr int SCR_F4 = scratch_bytes<P, TIO>() / 16;
  constexpr bool SP_LDS = P::spectra_in_lds(CH, NW, HERM, HP);
  constexpr int SPC_F4 = P::sp_f4(HERM);  // one channel's spectrum
  constexpr int SPL_F4 = SP_LDS ? P::spl_f4(CH, HERM) : 0;
  constexpr int TAB_F4 = K1 ? P::tab1_f4(HP) : P::tab_f4(HP), TWB_F4 = P::twb_f4(HP);
  constexpr int F0_H8 = K1 ? P::F0_H8 / 2 : P::F0_H8, F1_H8 = K1 ? P::F1_H8 / 2 : P::F1_H8;
  static_assert((TAB_F4 + SPL_F4 + NW * SCR_F4) * 16 <= 163840, "layout within the LDS of a CU");
  __shared__ float4 lds[TAB_F4 + SPL_F4 + NW * SCR_F4];
  h8* F0 = reinterpret_cast<h8*>(lds);
  h8* F1 = P::R1 == P::R0 ? F0 : F0 + F0_H8;
  float4* TW1 = lds + F0_H8 + F1_H8;
  float4* TW2 = P::TW_TABLES == 2 ? TW1 + TWB_F4 : TW1;
  float4* SPL = lds + TAB_F4;

  // the wavefront index is uniform: read it into a scalar register so the pair and
  // channel arithmetic derived from it runs on the scalar unit
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  TIO* S = reinterpret_cast<TIO*>(lds + TAB_F4 + SPL_F4 + wave * SCR_F4);
  const int BP = B >> 1, h0 = blockIdx.x * CH;
  const int nch = H - h0 < CH ? H - h0 : CH;  // channels of this workgroup

  // ---- tables and spectra: direct global -> LDS copies, issued first
  dma_to_lds<P::TW_TABLES * TWB_F4, NW>(TW1, [&](int k) { return twtab + k; }, lane, wave);
  if constexpr (CACHED) {
    // with K1 the first-kind runs only: LDS run i is table run 2i
    auto tab = [&](int R, int k) {
      return reinterpret_cast<const float4*>(ftab + cf_off(R) + (K1 ? ((k >> 6) << 7) + (k & 63) : k));
    };
    dma_to_lds<F0_H8, NW>(reinterpret_cast<float4*>(F0), [&](int k) { return tab(R0, k); }, lane, wave);
    if constexpr (P::R1 != P::R0)
      dma_to_lds<F1_H8, NW>(reinterpret_cast<float4*>(F1), [&](int k) { return tab(P::R1, k); }, lane, wave);
  }
  // channel h's spectrum (SPC_F4 float4) starts row h of the caller's [H][2L] complex64
  // buffer, whose rows are SP_F4 float4 apart
  if constexpr (SP_LDS) {
    // channel c of this workgroup goes to LDS slot c, the slots consecutive; what the
    // copy's whole runs add past the last channel repeats the last float4 of the last
    // channel (in bounds, never read)
    const int last = nch * SPC_F4 - 1;
    dma_to_lds<SPL_F4, NW>(SPL, [&](int k) {
      const int kk = k < last ? k : last, c = kk / SPC_F4;
      return kf + (size_t)(h0 + c) * P::SP_F4 + (kk - c * SPC_F4);
    }, lane, wave);
  }
  // spectrum of channel slot c: in LDS, or the channel's row in global memory
  auto spec = [&](int c) -> const float4* {
    if constexpr (SP_LDS) return SPL + c * SPC_F4;
    else return kf + (size_t)(h0 + c) * P::SP_F4;
  };
  if constexpr (!CACHED) {
    compute_dft<R0, 64 * NW, K1>(F0, tid);
    if constexpr (P::R1 != P::R0) compute_dft<P::R1, 64 * NW, K1>(F1, tid);
  }

  // ---- the first pairs. The waves of the first channel issue their loads right
  // after the copies: they follow them in the vector-memory queue, so waiting for all
  // but the last pair_load_issues() operations waits for the tables and spectra only
  // and the pair's data stays in flight across the barrier (a __syncthreads() would
  // drain it: its release fence waits for vmcnt 0). The other waves issue theirs
  // after the barrier, so the first channel's data lands (and is computed and
  // stored) while the rest is still in flight.
  const int npairs = nch * BP;
  PairLoads<P, TIO> cur;
  auto issue_first = [&]() {
    const int c = wave / BP, bp = wave - c * BP;
    const size_t ra = ((size_t)(2 * bp) * H + h0 + c) * P::L;
    issue_pair_loads<P, TIO>(u + ra, u + ra + (size_t)H * P::L, cur, lane);
  };
  const bool early = wave < BP && wave < npairs;
  __asm__ volatile("" ::: "memory");
  if (early) {
    issue_first();
#ifdef SFFFT_DEBUG_BARRIERS
    wait_vmcnt<0>();  // the pair's loads too: the barrier below then needs no count
#else
    wait_vmcnt<pair_load_issues<P, TIO>()>();
#endif
  } else {
    wait_vmcnt<0>();
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the in-kernel DFT fragments are written
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
  if (!early && wave < npairs) issue_first();

  // phase-2 fragments are read into VGPRs before the strip loop and held there (pinned,
  // rather than placed by the compiler) when there are at most two 16-wide tiles per
  // radix-R1 axis: 32 VGPRs, within the budget of three wavefronts per SIMD (64x32 with
  // 12 wavefronts: 150 VGPRs; measured 1-2% faster with bf16 I/O, equal with fp32)
  constexpr bool HOLD = P::MT <= 2;
  // fp32 input split into value and remainder where the launch is bound by its dispatch
  // floor and HBM, not by the SIMDs (L <= 512): removes the input's fp16 rounding, one of
  // the four roundings of a two-stage plan, for twice the phase-1 MFMAs (a quarter of
  // the pair's). bf16 samples are exact in fp16; the fp16-accumulation mode keeps the
  // one rounding.
  constexpr bool SPLIT = sizeof(TIO) == 4 && !ACC16 && P::L <= 512;
  if (wave < npairs) {
    const int c = wave / BP, bp = wave - c * BP;
    // 64x64: a SIMD's three wavefronts hold one pair of each channel, whose data lands
    // in channel order, and the last channel's compute sets the end of the launch. Its
    // wavefronts issue first (priority rising with the channel); the earlier channels
    // fill the issue slots it leaves. Alternating builds, two runs each, on two boxes:
    // fp32 I/O 30.6-31.0 -> 29.3-29.4 us and 29.0-29.1 -> 28.7-28.9, bf16 25.1 -> 24.7-24.8
    // and 24.0 -> 23.7-23.9, bf16 with fp16 accumulation 24.3 -> 23.2 and 23.4-23.7 ->
    // 22.5-22.7 (outputs bit-identical). fp32 I/O with fp16 accumulation went 30.0 -> 33.0
    // and keeps one level. 64x32 (L = 1024), three runs each: bf16 with fp16 accumulation
    // 10.83-10.95 -> 10.32-10.58 us; bf16 unchanged (11.95-12.08 against 11.96-11.98) and
    // fp32 with fp16 accumulation 5% slower, so only the first takes it.
    if constexpr ((P::R0 == 64 && P::R1 == 64 && !(HP && sizeof(TIO) == 4)) ||
                  (P::R0 == 64 && P::R1 == 32 && HP && sizeof(TIO) == 2)) {
      if (c == 1) __builtin_amdgcn_s_setprio(1);
      else if (c >= 2) __builtin_amdgcn_s_setprio(2);
    }
    const size_t ra = ((size_t)(2 * bp) * H + h0 + c) * P::L, rb = ra + (size_t)H * P::L;
    process_pair<P, TIO, ACC16, HOLD, K1, HERM, SPLIT, HP>(cur, S, spec(c), y + ra, y + rb, F0, F1, TW1, TW2, lane);
  }
  for (int p = wave + NW; p < npairs; p += NW) {
    // compiler-only barrier: keeps the table reads inside the loop (hoisting them
    // would pin every twiddle tile in VGPRs)
    __asm__ volatile("" ::: "memory");
    // the lane index is made opaque per iteration, so the per-lane addresses derived
    // from it are recomputed here instead of being hoisted out of the loop and kept
    // live (or spilled) across it
    int ln = lane;
    __asm__ volatile("" : "+v"(ln));
    // 64x64 only: known to be a lane index again, its row-chunk masks fold (144 instead of
    // 168 VGPRs in the fp16-accumulation instantiation). In the other plans the same mask
    // raised the allocation, to a spill of 8-28 values at 64x32.
    if constexpr (P::R0 == 64 && P::R1 == 64) ln &= 63;
    const int c = p / BP, bp = p - c * BP;
    const size_t ra = ((size_t)(2 * bp) * H + h0 + c) * P::L, rb = ra + (size_t)H * P::L;
    issue_pair_loads<P, TIO>(u + ra, u + rb, cur, ln);
    process_pair<P, TIO, ACC16, HOLD, K1, HERM, SPLIT, HP>(cur, S, spec(c), y + ra, y + rb, F0, F1, TW1, TW2, ln);
  }
}

}  // namespace sffft
