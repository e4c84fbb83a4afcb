// gfx950 (CDNA4) kernels of the paged tree-decode attention path.
//
// attend16 / attend32: a workgroup of four wave64s runs one task, either
//   - up to four wave items: each wave alone attends its item (<= 16 query
//     rows, i.e. one sequence's GQA group of a private tail, or a few
//     sequences of a small shared segment) over the item's pages, with the
//     next page pair's loads in flight behind the current pair's math; or
//   - one group item (<= 128 rows, a tree-shared prefix; 64 at head_dim 256
//     and with FP8 KV): every wave owns up to 32 rows and all four consume
//     the same page pairs, which the workgroup stages once into LDS (16-bit
//     KV: direct global->LDS loads into a ring of page pairs; FP8 / MXFP8:
//     through registers, double-buffered), so a shared page is fetched once
//     per 128 rows instead of once per wave.
// Each wave keeps an online softmax for its rows and writes one partial
// state per row.  ReferenceBackend::decode (crates/dendrite-core/src/
// attention/backend.rs:206-265) computes softmax(q K^T * scale) V over the
// concatenated pages; this is the same quantity, split over pages and merged
// exactly by log-sum-exp.
//
// Matrix-core mapping (lane l = 16*g + c, g = l / 16, c = l % 16):
//   S^T = K . Q^T with v_mfma_f32_16x16x32_{bf16,f16}: A = 16 tokens x 32 dims
//   of one page (lane holds token c, 8 consecutive dims), B = 32 dims x 16 query
//   rows (lane holds row c, the same 8 dims).  The accumulator gives lane
//   (g, c) the scores of row c for tokens 4g..4g+3.
//   O^T += V^T . P^T with the same instruction over two pages (32 tokens): the
//   B operand (P^T) is exactly the two pages' score accumulators of the lane
//   after exp2, so the probabilities never leave registers.  The A operand
//   (V^T) holds, for d-block e, V[token][c*EPL + e] for the lane's 8 tokens,
//   built by byte permutes from 16-byte row loads (EPL = head_dim / 16).
//   Lane (g, c) ends up holding O[row c][4g*EPL .. 4g*EPL + 4*EPL).
//   (The LDS path of group items builds V^T with transposing LDS reads
//   instead, and its lanes hold O[row c][16e + 4g + i]; see there.)
// FP8 E4M3 pages are converted to bf16 in registers (exact: E4M3 is a subset
// of bf16); the per-(page, head) fp32 scale multiplies the scores (K) and the
// probabilities (V), which equals dequantising every element.  MXFP8 pages
// are converted with their E8M0 group scale by v_cvt_scalef32_pk_bf16_fp8
// (exact: power-of-two scaling).
#include <hip/hip_runtime.h>
#include <math.h>
#include <type_traits>
#include "dh_device.hpp"
#include "dendrite_hip.h"

namespace dh {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f2 __attribute__((ext_vector_type(2)));

constexpr uint32_t KVF_F16 = 0, KVF_BF16 = 1, KVF_F32 = 2, KVF_FP8 = 3, KVF_MX = 4;
constexpr float kNegInf = -__builtin_inff();

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Max over the four lanes l, l^16, l^32, l^48 (the four 16-lane rows of the
// wave) with the gfx950 permlane swaps: after swap(x, x) the two results hold
// x of the lane and of its partner row, so the max of the pair is the
// xor-16 / xor-32 reduction without a trip through the LDS crossbar.
__device__ __forceinline__ float rowgroup_max(float x) {
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float rowgroup_sum(float x) {
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Load n dwords (n in {1, 2, 4, 8}) from a naturally aligned address.
template <int N>
__device__ __forceinline__ void load_dwords(uint32_t* dst, const void* src) {
    if constexpr (N == 1) {
        dst[0] = *reinterpret_cast<const uint32_t*>(src);
    } else if constexpr (N == 2) {
        u32x2 v = *reinterpret_cast<const u32x2*>(src);
        dst[0] = v.x; dst[1] = v.y;
    } else {
        #pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            u32x4 v = reinterpret_cast<const u32x4*>(src)[i];
            dst[4 * i + 0] = v.x; dst[4 * i + 1] = v.y;
            dst[4 * i + 2] = v.z; dst[4 * i + 3] = v.w;
        }
    }
}

// E8M0 scale byte -> float 2^(e-127); 255 -> NaN (OCP MX v1.0).
__device__ __forceinline__ float e8m0_to_float(uint32_t e) {
    uint32_t bits = e == 0 ? 0x00400000u : (e == 255 ? 0x7FC00000u : (e << 23));
    return __uint_as_float(bits);
}

// Four E4M3 bytes -> four bf16 (two dwords), multiplied by sc (a power of two).
__device__ __forceinline__ void e4m3x4_to_bf16(uint32_t x, float sc, uint32_t& lo, uint32_t& hi) {
    bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x, sc, false);
    bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x, sc, true);
    lo = __builtin_bit_cast(uint32_t, a);
    hi = __builtin_bit_cast(uint32_t, b);
}

// The same into f16 (H) or bf16: 8-bit pools under f16 queries compute in
// f16 (every E4M3 code is exact in f16; code x scale rounds once).
template <bool H>
__device__ __forceinline__ void e4m3x4_cvt(uint32_t x, float sc, uint32_t& lo, uint32_t& hi) {
    if constexpr (H) {
        f16x2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, sc, false);
        f16x2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, sc, true);
        lo = __builtin_bit_cast(uint32_t, a);
        hi = __builtin_bit_cast(uint32_t, b);
    } else {
        e4m3x4_to_bf16(x, sc, lo, hi);
    }
}

__device__ __forceinline__ uint32_t pack2(float a, float b, bool f16) {
    if (f16) {
        f16x2 t = {(_Float16)a, (_Float16)b};
        return __builtin_bit_cast(uint32_t, t);
    }
    bf16x2 t = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, t);
}

__device__ __forceinline__ float unpack_lo(uint32_t v, bool f16) {
    if (f16) return float(__builtin_bit_cast(f16x2, v)[0]);
    return __uint_as_float(v << 16);
}

__device__ __forceinline__ float unpack_hi(uint32_t v, bool f16) {
    if (f16) return float(__builtin_bit_cast(f16x2, v)[1]);
    return __uint_as_float(v & 0xFFFF0000u);
}

template <bool F16>
__device__ __forceinline__ f4 mma16(const uint32_t* a, const uint32_t* b, f4 c) {
    u32x4 av = {a[0], a[1], a[2], a[3]};
    u32x4 bv = {b[0], b[1], b[2], b[3]};
    if constexpr (F16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av),
                                                      __builtin_bit_cast(f16x8, bv), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av),
                                                       __builtin_bit_cast(bf16x8, bv), c, 0, 0, 0);
    }
}

// acc *= alpha in place.  The rescale runs on a rarely taken branch; done
// through "+v" operands the accumulator keeps its registers on both paths,
// so the compiler needs no copies of the accumulators to merge the paths.
__device__ __forceinline__ void scale_inplace(f4& acc, float alpha) {
    float x = acc[0], y = acc[1], z = acc[2], w = acc[3];
    asm volatile("v_mul_f32 %0, %0, %4\n\tv_mul_f32 %1, %1, %4\n\tv_mul_f32 %2, %2, %4\n\tv_mul_f32 %3, %3, %4"
                 : "+v"(x), "+v"(y), "+v"(z), "+v"(w)
                 : "v"(alpha));
    acc = f4{x, y, z, w};
}

// Query head served by row rho of an item (GQA mapping per dh_gqa_mapping).
__device__ __forceinline__ void row_target(const AttendArgs& a, const Item& it, uint32_t row,
                                           uint32_t& seq, uint32_t& slot, uint32_t& qh) {
    uint32_t rho = it.row_begin + row;
    uint32_t sl = rho / a.r;
    uint32_t j = rho - sl * a.r;
    SeqSlot ss = a.seqslots[it.seq_off + sl];
    seq = ss.seq;
    slot = ss.slot;
    qh = a.gqa_tiled ? it.kv_head + j * a.hkv : it.kv_head * a.r + j;
}

// Group items of the launch: the plan's count, or on the CSR path what the
// CSR planning kernel of this call wrote (its group items come first).
__device__ __forceinline__ uint32_t group_item_count(const AttendArgs& a) {
    return a.csr_hdr ? __builtin_amdgcn_readfirstlane(a.csr_hdr[4]) : a.n_group_items;
}

// Item of wave `wave` in a workgroup past the ng group items (AttendArgs):
// on the plan path an index into the items (group items first), on the CSR
// path the wave item's own number (csr_item).
__device__ __forceinline__ uint32_t wave_item_index(const AttendArgs& a, int wave, uint32_t ng) {
    return (a.csr_hdr ? 0u : ng) + (blockIdx.x - ng) * kWaves + uint32_t(wave);
}

// Wave items on the plan path: the plan's count; on the CSR path: what the
// CSR planning kernel of this call wrote (its nodes' wave items, then one
// per chunk of each sequence's own pages).
__device__ __forceinline__ uint32_t wave_item_end(const AttendArgs& a) {
    return a.csr_hdr ? __builtin_amdgcn_readfirstlane(a.csr_hdr[1]) + __builtin_amdgcn_readfirstlane(a.csr_hdr[6])
                     : a.n_group_items + a.n_wave_items;
}

// Wave item idx of a CSR call: the cascade's node wave items (stored after
// its ng group items in a.items), then the items derived from the tables.
__device__ __forceinline__ Item csr_wave_item(const AttendArgs& a, uint32_t idx, uint32_t ng);

// Wave item idx of a CSR call, derived from the tables: idx = (j * hkv +
// kv_head) * nrb + row block; seqslots[j] names the j-th chunk in dispatch
// order, chunk k of sequence b in slot slot_ptr[b] + G + k, pages
// indptr[b] + L + k * chunk .. (the last chunk ends at b's last page), where
// b's first L pages are read by group items into its first G slots (csr_skip;
// L = G = 0 without a cascade).  seq_off = j: the row's slot is read back from
// seqslots[j] (row_target).
__device__ __forceinline__ Item csr_item(const AttendArgs& a, uint32_t idx) {
    const uint32_t nrb = a.csr_nrb, per = a.hkv * nrb;
    const uint32_t j = idx / per, rem = idx - j * per;
    const uint32_t h = rem / nrb, rb = rem - h * nrb;
    const uint32_t b = __builtin_amdgcn_readfirstlane(a.seqslots[j].seq);
    const uint32_t slot = __builtin_amdgcn_readfirstlane(a.seqslots[j].slot);
    const uint32_t chunk = __builtin_amdgcn_readfirstlane(a.csr_hdr[0]);
    const uint32_t skip = a.csr_skip ? __builtin_amdgcn_readfirstlane(a.csr_skip[b]) : 0u;
    const uint32_t k = slot - __builtin_amdgcn_readfirstlane(a.csr_slot_ptr[b]) - (skip >> 16);
    const uint32_t p0 = uint32_t(__builtin_amdgcn_readfirstlane(a.csr_indptr[b])) + (skip & 0xFFFFu);
    const uint32_t n = uint32_t(__builtin_amdgcn_readfirstlane(a.csr_indptr[b + 1])) - p0;
    Item it;
    it.page_off = p0 + k * chunk;
    it.npages = min(chunk, n - k * chunk);
    it.seq_off = j;
    it.row_begin = rb * kWaveRows;
    it.nrows = min(uint32_t(kWaveRows), a.r - rb * kWaveRows);
    it.kv_head = h;
    it.flags = (k + 1) * chunk >= n ? kItemTail : 0u;
    it.tail_seq = b;
    return it;
}

__device__ __forceinline__ Item csr_wave_item(const AttendArgs& a, uint32_t idx, uint32_t ng) {
    const uint32_t nw = __builtin_amdgcn_readfirstlane(a.csr_hdr[6]);
    return idx < nw ? a.items[ng + idx] : csr_item(a, idx - nw);
}

// Valid tokens of page index i of an item.
__device__ __forceinline__ int page_tokens(const Item& it, uint32_t i, int last_len) {
    if (i >= it.npages) return 0;
    return ((it.flags & kItemTail) && i + 1 == it.npages) ? last_len : kPageSize;
}

// Tokens in the item's last page.  Read through readfirstlane: the value is
// wave-uniform, and telling the compiler so keeps every branch on the page
// fill (full pair / partial pair) a scalar branch instead of a masked
// execution of both sides.
__device__ __forceinline__ int item_last_len(const AttendArgs& a, const Item& it) {
    if (!(it.flags & kItemTail)) return kPageSize;
    int L;
    if (a.last_page_len)
        L = __builtin_amdgcn_readfirstlane(a.last_page_len[it.tail_seq]);
    else if (a.lpl_inline)   // 4 bits a sequence in the kernel arguments, 0 for 16
        L = int((__builtin_amdgcn_readfirstlane(a.lpl_nib[it.tail_seq >> 3]) >> (4 * (it.tail_seq & 7))) & 15u);
    else
        return kPageSize;
    return (L <= 0 || L > kPageSize) ? kPageSize : L;
}

// Partial states: fp32 for f32 queries; otherwise f16, each row scaled by a
// power of two 2^-k chosen from the row's largest magnitude (below 2^15
// after scaling), so f16's range never clips and its 11-bit significand
// holds every row at the same relative precision whatever the magnitude of
// V.  k goes with the row's log2-sum-exp (PartialLse); the merge folds 2^k
// into the row's weight, which is exact.
__device__ __forceinline__ int partial_exp(float row_max_abs) {
    if (!(row_max_abs > 0.f) || !(row_max_abs < 3.0e38f)) return 0;
    return max(__builtin_amdgcn_frexp_expf(row_max_abs) - 15, -100);   // row_max_abs < 2^(k + 15)
}

template <int N>
__device__ __forceinline__ void store_u32s(uint16_t* p, const uint32_t (&v)[N]) {
    if constexpr (N % 4 == 0) {
        #pragma unroll
        for (int k = 0; k < N; k += 4)
            *reinterpret_cast<u32x4*>(p + 2 * k) = u32x4{v[k], v[k + 1], v[k + 2], v[k + 3]};
    } else if constexpr (N == 2) {
        *reinterpret_cast<u32x2*>(p) = u32x2{v[0], v[1]};
    } else {
        static_assert(N == 1, "store width");
        *reinterpret_cast<uint32_t*>(p) = v[0];
    }
}

// Writes the partial states of one wave's rows: tiles rt < nrt, row
// row0 + 16*rt + c of the item, to partial rows dst[rt].  O[rt][e][i] is
// element d = (4g+i)*EPL + e.  lrow[rt]: the row's total weight when
// ROW_SUMMED, else this lane's share (summed over the row's four lanes here).
template <int D, int RT, bool ROW_SUMMED, bool F32>
__device__ __forceinline__ void write_wave_partial(const AttendArgs& a, const Item& it, uint32_t row0,
                                                   int nrt, const uint32_t (&dst)[RT], const float (&m)[RT],
                                                   const float (&lrow)[RT], const f4 (&O)[RT][D / 16], int g,
                                                   int c) {
    constexpr int EPL = D / 16;
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        if (rt >= nrt) break;
        const float lt = ROW_SUMMED ? lrow[rt] : rowgroup_sum(lrow[rt]);
        const uint32_t row = row0 + rt * kTileRows + c;
        const float inv = lt > 0.f ? 1.f / lt : 0.f;
        int k = 0;
        if constexpr (!F32) {
            float mx = 0.f;
            #pragma unroll
            for (int e = 0; e < EPL; ++e)
                #pragma unroll
                for (int i = 0; i < 4; ++i) mx = fmaxf(mx, fabsf(O[rt][e][i]));
            k = partial_exp(rowgroup_max(mx) * inv);
        }
        if (row < it.nrows) {
            if constexpr (F32) {
                float* o = static_cast<float*>(a.ws_o) + uint64_t(dst[rt]) * D;
                #pragma unroll
                for (int i = 0; i < 4; ++i) {
                    #pragma unroll
                    for (int e = 0; e < EPL; e += 4) {
                        f4 v = {O[rt][e][i] * inv, O[rt][e + 1][i] * inv, O[rt][e + 2][i] * inv,
                                O[rt][e + 3][i] * inv};
                        *reinterpret_cast<f4*>(o + (4 * g + i) * EPL + e) = v;
                    }
                }
            } else {
                const float sc = __builtin_amdgcn_ldexpf(inv, -k);
                uint16_t* o = static_cast<uint16_t*>(a.ws_o) + uint64_t(dst[rt]) * D;
                #pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint32_t v[EPL / 2];
                    #pragma unroll
                    for (int e = 0; e < EPL; e += 2) v[e / 2] = pack2(O[rt][e][i] * sc, O[rt][e + 1][i] * sc, true);
                    store_u32s<EPL / 2>(o + (4 * g + i) * EPL, v);
                }
            }
            if (g == 0) a.ws_lse[dst[rt]] = PartialLse{lt > 0.f ? m[rt] + log2f(lt) : kNegInf, float(k)};
        }
    }
}

// Query rows of NRT tiles as B operands: lane (g, c) holds row row0+16*rt+c,
// dims kb*32 + 8g .. +8 (zero for rows outside the item).  K16: the order
// of 8-bit K rows loaded in 16-byte pieces (load_page_k): k-block kb = 2j + h
// holds dims 64j + 16g + 8h .. +8.  A dot product does not depend on the
// order of its terms, so K and q only have to agree on it.
template <int D, int RT, bool K16 = false>
__device__ __forceinline__ void load_q16(const AttendArgs& a, const Item& it, uint32_t row0, int nrt,
                                         uint32_t (&qB)[RT][D / 32][4], uint32_t (&dst)[RT], int g, int c) {
    constexpr int KB = D / 32;
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const uint32_t row = row0 + rt * kTileRows + c;
        dst[rt] = 0u;
        if (rt < nrt && row < it.nrows) {
            uint32_t seq, slot, qh;
            row_target(a, it, row, seq, slot, qh);
            dst[rt] = slot * a.hq + qh;
            const uint16_t* qp = reinterpret_cast<const uint16_t*>(a.q) + (uint64_t(seq) * a.hq + qh) * D;
            #pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                load_dwords<4>(qB[rt][kb], qp + (K16 ? 64 * (kb >> 1) + 16 * g + 8 * (kb & 1) : kb * 32 + 8 * g));
                #pragma unroll
                for (int i = 0; i < 4; ++i) qB[rt][kb][i] ^= a.q_sign;
            }
        } else {
            #pragma unroll
            for (int kb = 0; kb < KB; ++kb) qB[rt][kb][0] = qB[rt][kb][1] = qB[rt][kb][2] = qB[rt][kb][3] = 0u;
        }
    }
}

// ---------------------------------------------------------------- pair math
// Scores of a page pair for NRT row tiles: s[rt][p] = S^T tile of page p
// (k0 / k1: the two pages' K operands).
template <int D, bool F16, int NRT, int RT>
__device__ __forceinline__ void pair_scores(const uint32_t (&k0)[D / 32][4], const uint32_t (&k1)[D / 32][4],
                                            const uint32_t (&qB)[RT][D / 32][4], f4 (&s)[RT][2]) {
    constexpr int KB = D / 32;
    #pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
        s[rt][0] = f4{0.f, 0.f, 0.f, 0.f};
        s[rt][1] = f4{0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            s[rt][0] = mma16<F16>(k0[kb], qB[rt][kb], s[rt][0]);
            s[rt][1] = mma16<F16>(k1[kb], qB[rt][kb], s[rt][1]);
        }
    }
}

// Online softmax of a pair's scores and O^T += V^T P^T.  f0/f1: scale_log2
// times the pages' K scales; v0s/v1s: the pages' V scales (1 unless FP8
// block-scaled); n0/n1: valid tokens of the two pages (n1 = 0: no page).
// v0 / v1 hold, per page, the V rows of tokens 4g+j (bf16/f16 dwords, zero
// for invalid tokens).
//
// Running max: a row's reference max m only moves when some score exceeds it
// by more than kLazy (so every exp2 stays <= 2^kLazy).  Whether that happens
// is decided from each lane's own scores and a ballot; the cross-lane max and
// the O rescale run only then, which after the first pairs is rare.
// Row sum: one more MFMA per tile multiplies the rounded probabilities by an
// all-ones A operand, so L holds, in every lane of row c, the sum of exactly
// the weights the PV MFMAs used (O / L is then a convex combination of V rows
// whatever the rounding of P).
template <int D, bool F16, int NRT, int RT, bool BLOCK_SCALE>
__device__ __forceinline__ void pair_softmax(const f4 (&s)[RT][2], int n0, int n1, float f0, float f1,
                                             float v0s, float v1s, float (&m)[RT], f4 (&L)[RT],
                                             f4 (&O)[RT][D / 16], int g, uint32_t (&pB)[RT][4]) {
    constexpr int EPL = D / 16;
    constexpr float kLazy = 8.f;                  // running-max slack (log2 units)
    const uint32_t one2 = F16 ? 0x3C003C00u : 0x3F803F80u;
    const uint32_t ones[4] = {one2, one2, one2, one2};
    const bool full = (n0 == kPageSize) && (n1 == kPageSize);
    #pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
        float x0[4], x1[4];
        #pragma unroll
        for (int i = 0; i < 4; ++i) {
            x0[i] = s[rt][0][i];
            x1[i] = s[rt][1][i];
        }
        if (!full) {
            #pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (4 * g + i >= n0) x0[i] = kNegInf;
                if (4 * g + i >= n1) x1[i] = kNegInf;
            }
        }
        // Lane-local max over raw scores: the scale factors are positive
        // (scale_log2 > 0; FP8 block scales are checked on write).
        const float r0 = fmaxf(fmaxf(x0[0], x0[1]), fmaxf(x0[2], x0[3]));
        const float r1 = fmaxf(fmaxf(x1[0], x1[1]), fmaxf(x1[2], x1[3]));
        const float lm = fmaxf(r0 * f0, r1 * f1);          // -inf * f stays -inf
        if (__ballot(lm > m[rt] + kLazy)) {
            const float mx = rowgroup_max(lm);
            const float mnew = mx > m[rt] + kLazy ? mx : m[rt];
            const float alpha = (m[rt] == kNegInf) ? 0.f : fast_exp2(m[rt] - mnew);
            m[rt] = mnew;
            scale_inplace(L[rt], alpha);
            #pragma unroll
            for (int e = 0; e < EPL; ++e) scale_inplace(O[rt][e], alpha);
        }
        const float nm = (m[rt] == kNegInf) ? 0.f : -m[rt];
        #pragma unroll
        for (int i = 0; i < 4; ++i) {
            x0[i] = fast_exp2(__builtin_fmaf(x0[i], f0, nm));
            x1[i] = fast_exp2(__builtin_fmaf(x1[i], f1, nm));
        }
        uint32_t pk[4];
        pk[0] = pack2(x0[0], x0[1], F16);
        pk[1] = pack2(x0[2], x0[3], F16);
        pk[2] = pack2(x1[0], x1[1], F16);
        pk[3] = pack2(x1[2], x1[3], F16);
        L[rt] = mma16<F16>(ones, pk, L[rt]);
        if constexpr (BLOCK_SCALE) {
            pB[rt][0] = pack2(unpack_lo(pk[0], F16) * v0s, unpack_hi(pk[0], F16) * v0s, F16);
            pB[rt][1] = pack2(unpack_lo(pk[1], F16) * v0s, unpack_hi(pk[1], F16) * v0s, F16);
            pB[rt][2] = pack2(unpack_lo(pk[2], F16) * v1s, unpack_hi(pk[2], F16) * v1s, F16);
            pB[rt][3] = pack2(unpack_lo(pk[3], F16) * v1s, unpack_hi(pk[3], F16) * v1s, F16);
        } else {
            #pragma unroll
            for (int k = 0; k < 4; ++k) pB[rt][k] = pk[k];
        }
    }
}

template <int D, bool F16, int NRT, int RT, bool BLOCK_SCALE>
__device__ __forceinline__ void pair_softmax_pv(const f4 (&s)[RT][2], const uint32_t (&v0)[4][D / 32],
                                                const uint32_t (&v1)[4][D / 32],
                                                int n0, int n1, float f0, float f1, float v0s, float v1s,
                                                float (&m)[RT], f4 (&L)[RT], f4 (&O)[RT][D / 16], int g) {
    constexpr int EPL = D / 16;
    uint32_t pB[RT][4];
    pair_softmax<D, F16, NRT, RT, BLOCK_SCALE>(s, n0, n1, f0, f1, v0s, v1s, m, L, O, g, pB);
    // The V operand of a d-block (element e of the lane's 8 tokens) is
    // shared by all row tiles.
    #pragma unroll
    for (int e = 0; e < EPL; ++e) {
        const int w = e >> 1;
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
        uint32_t vA[4];
        vA[0] = __builtin_amdgcn_perm(v0[1][w], v0[0][w], sel);
        vA[1] = __builtin_amdgcn_perm(v0[3][w], v0[2][w], sel);
        vA[2] = __builtin_amdgcn_perm(v1[1][w], v1[0][w], sel);
        vA[3] = __builtin_amdgcn_perm(v1[3][w], v1[2][w], sel);
        #pragma unroll
        for (int rt = 0; rt < NRT; ++rt) O[rt][e] = mma16<F16>(vA, pB[rt], O[rt][e]);
    }
}

// Zeroes, in a lane's 16-bit V rows (tokens 4g+j), the tokens at or past
// nt (their probabilities are zero; garbage there must not reach O).
template <int D>
__device__ __forceinline__ void mask_v_rows(uint32_t (&v)[4][D / 32], int g, int nt) {
    #pragma unroll
    for (int j = 0; j < 4; ++j) {
        const bool ok = 4 * g + j < nt;
        #pragma unroll
        for (int w = 0; w < D / 32; ++w) v[j][w] = ok ? v[j][w] : 0u;
    }
}

// ------------------------------------------------------------- wave items
// Raw pool bytes of one page for this lane (K rows of token c, V rows of
// tokens 4g..4g+3), plus the MX scale bytes that go with them.
template <int D, uint32_t KVF>
struct PageRaw {
    static constexpr bool FP8 = (KVF == KVF_FP8 || KVF == KVF_MX);
    static constexpr int KB = D / 32;
    static constexpr int EPL = D / 16;
    static constexpr int KW = FP8 ? 2 : 4;           // dwords per k-chunk
    static constexpr int VW = FP8 ? EPL / 4 : EPL / 2;
    static constexpr int G = D / 32;                 // MX groups per token
    uint32_t k[KB][KW];
    uint32_t v[4][VW];
    uint32_t ksc[KVF == KVF_MX ? G : 1];            // MX: K scale byte per k-chunk
    uint32_t vsc[KVF == KVF_MX ? 4 : 1];            // MX: V scale byte per token j
};

template <int D, uint32_t KVF>
__device__ __forceinline__ void load_page_k(PageRaw<D, KVF>& r, const AttendArgs& a, uint32_t page,
                                            uint32_t head, int g, int c) {
    using R = PageRaw<D, KVF>;
    constexpr int EB = R::FP8 ? 1 : 2;
    const uint8_t* kp = a.kv + plane_offset(page, 0, head, a.hkv, D, EB);
    if constexpr (R::FP8) {
        // 16 codes (16 bytes) per lane: dims 64j + 16g .. +16 of token c
        // feed k-blocks 2j and 2j + 1 (the query is loaded in the same
        // order), so a load instruction reads 64-byte runs of 16 rows
        // instead of 32-byte ones.
        #pragma unroll
        for (int j = 0; j < R::KB / 2; ++j) {
            uint32_t t[4];
            load_dwords<4>(t, kp + c * D + 64 * j + 16 * g);
            r.k[2 * j][0] = t[0];
            r.k[2 * j][1] = t[1];
            r.k[2 * j + 1][0] = t[2];
            r.k[2 * j + 1][1] = t[3];
        }
    } else {
        #pragma unroll
        for (int kb = 0; kb < R::KB; ++kb)
            load_dwords<R::KW>(r.k[kb], kp + (c * D + kb * 32 + 8 * g) * EB);
    }
    if constexpr (KVF == KVF_MX) {
        // the MX group (32 dims) of k-block 2j + h's codes is 2j + g / 2
        const uint8_t* s = reinterpret_cast<const uint8_t*>(a.scales) +
                           ((uint64_t(page) * 2 + 0) * a.hkv + head) * uint64_t(kPageSize) * R::G;
        #pragma unroll
        for (int kb = 0; kb < R::G; ++kb) r.ksc[kb] = s[c * R::G + 2 * (kb >> 1) + (g >> 1)];
    }
}

template <int D, uint32_t KVF>
__device__ __forceinline__ void load_page_v(PageRaw<D, KVF>& r, const AttendArgs& a, uint32_t page,
                                            uint32_t head, int g, int c) {
    using R = PageRaw<D, KVF>;
    constexpr int EB = R::FP8 ? 1 : 2;
    const uint8_t* vp = a.kv + plane_offset(page, 1, head, a.hkv, D, EB);
    #pragma unroll
    for (int j = 0; j < 4; ++j)
        load_dwords<R::VW>(r.v[j], vp + ((4 * g + j) * D + c * R::EPL) * EB);
    if constexpr (KVF == KVF_MX) {
        const uint8_t* s = reinterpret_cast<const uint8_t*>(a.scales) +
                           ((uint64_t(page) * 2 + 1) * a.hkv + head) * uint64_t(kPageSize) * R::G;
        #pragma unroll
        for (int j = 0; j < 4; ++j) r.vsc[j] = s[(4 * g + j) * R::G + (c * R::EPL) / 32];
    }
}

// K rows of a page as MFMA A operands (bf16/f16 dwords; 8-bit codes into
// f16 when H).
template <int D, uint32_t KVF, bool H>
__device__ __forceinline__ void k_operand(const PageRaw<D, KVF>& r, uint32_t (&op)[D / 32][4]) {
    using R = PageRaw<D, KVF>;
    #pragma unroll
    for (int kb = 0; kb < R::KB; ++kb) {
        if constexpr (!R::FP8) {
            #pragma unroll
            for (int w = 0; w < 4; ++w) op[kb][w] = r.k[kb][w];
        } else {
            const float sc = KVF == KVF_MX ? e8m0_to_float(r.ksc[kb]) : 1.f;
            e4m3x4_cvt<H>(r.k[kb][0], sc, op[kb][0], op[kb][1]);
            e4m3x4_cvt<H>(r.k[kb][1], sc, op[kb][2], op[kb][3]);
        }
    }
}

// V rows of a page (tokens 4g+j, dims c*EPL..) as bf16/f16 dwords; rows of
// tokens at or beyond nt are zero so that garbage past the valid tokens can
// never reach the accumulator (their probabilities are zero).
template <int D, uint32_t KVF, bool H>
__device__ __forceinline__ void v_operand(const PageRaw<D, KVF>& r, int g, int nt,
                                          uint32_t (&op)[4][D / 32]) {
    using R = PageRaw<D, KVF>;
    #pragma unroll
    for (int j = 0; j < 4; ++j) {
        const bool ok = 4 * g + j < nt;
        if constexpr (!R::FP8) {
            #pragma unroll
            for (int w = 0; w < R::VW; ++w) op[j][w] = ok ? r.v[j][w] : 0u;
        } else {
            const float sc = KVF == KVF_MX ? e8m0_to_float(r.vsc[j]) : 1.f;
            #pragma unroll
            for (int w = 0; w < R::VW; ++w)
                e4m3x4_cvt<H>(ok ? r.v[j][w] : 0u, sc, op[j][2 * w], op[j][2 * w + 1]);
        }
    }
}

// One wave attends a wave item (one tile of <= 16 rows) over all its pages.
// The next pair's K is requested as soon as the score MFMAs have consumed K,
// its V as soon as the PV MFMAs have consumed V, so the loads of pair i+1 are
// in flight behind the math of pair i without a second register buffer.
// Past the end the loads repeat the last page: issuing them unconditionally
// keeps one load order on every path, so the wait before a pair's scores
// covers K only.
template <int D, uint32_t KVF, bool F16>
__device__ __forceinline__ void wave_item(const AttendArgs& a, const Item& it, int g, int c) {
    constexpr int EPL = D / 16;
    constexpr int KB = D / 32;
    constexpr bool BLOCK_SCALE = (KVF == KVF_FP8);
    uint32_t qB[1][KB][4];
    uint32_t dst[1];
    load_q16<D, 1, PageRaw<D, KVF>::FP8>(a, it, 0, 1, qB, dst, g, c);
    float m[1] = {kNegInf};
    f4 L[1] = {f4{0.f, 0.f, 0.f, 0.f}};
    f4 O[1][EPL];
    #pragma unroll
    for (int e = 0; e < EPL; ++e) O[0][e] = f4{0.f, 0.f, 0.f, 0.f};

    const int last_len = item_last_len(a, it);
    const uint32_t head = it.kv_head;
    const uint32_t np = it.npages;
    const float* bsc = reinterpret_cast<const float*>(a.scales);
    // The item's page ids in registers (lane l holds ids l, l + 64, ...), so
    // a refill needs no memory round trip of its own: a load issued just
    // before a refill would be the newest outstanding one, and waiting for it
    // would also drain the page loads in flight.
    const int lane = 16 * g + c;
    uint32_t idv[kWaveIdRegs];
    bool bad = false;
    #pragma unroll
    for (int k = 0; k < kWaveIdRegs; ++k) {
        const uint32_t i = uint32_t(lane + 64 * k);
        idv[k] = i < np ? a.pages[it.page_off + i] : 0u;
        bad |= idv[k] >= a.page_limit;
        idv[k] = idv[k] < a.page_limit ? idv[k] : 0u;
    }
    if (__ballot(bad) && a.seq_bad && lane == 0) a.seq_bad[it.tail_seq] = 1u;
    auto page_id = [&](uint32_t i) -> uint32_t {
        i = i < np ? i : np - 1;
        uint32_t r = 0;
        #pragma unroll
        for (int k = 0; k < kWaveIdRegs; ++k)
            if ((i >> 6) == uint32_t(k)) r = __builtin_amdgcn_readlane(idv[k], int(i & 63));
        return r;
    };

    // DEPTH page pairs in flight: buffer p % DEPTH holds pair p; once pair
    // p's K (then V) has been consumed, its K (V) registers take pair
    // p + DEPTH's.  Two for E4M3 pages at head_dim <= 128 (a pair is 32
    // registers).  16-bit pages keep one: two fit in registers at head_dim
    // 128, but on C3 the extra traffic of the tails slowed the shared-prefix
    // items beside them more than it sped the tails (30.4 against 29.2 µs).
    constexpr int DEPTH = (KVF == KVF_FP8 && D <= 128) ? 2 : 1;
    PageRaw<D, KVF> pr[DEPTH][2];
    float ks[DEPTH][2], vs[DEPTH][2];
    #pragma unroll
    for (int d = 0; d < DEPTH; ++d) ks[d][0] = ks[d][1] = vs[d][0] = vs[d][1] = 1.f;
    auto load_pair = [&](int buf, uint32_t pair, bool kpart) {
        #pragma unroll
        for (int p = 0; p < 2; ++p) {
            const uint32_t pg = page_id(2 * pair + p);
            if (kpart) {
                load_page_k<D, KVF>(pr[buf][p], a, pg, head, g, c);
                if constexpr (BLOCK_SCALE) ks[buf][p] = bsc[(uint64_t(pg) * 2 + 0) * a.hkv + head];
            } else {
                load_page_v<D, KVF>(pr[buf][p], a, pg, head, g, c);
                if constexpr (BLOCK_SCALE) vs[buf][p] = bsc[(uint64_t(pg) * 2 + 1) * a.hkv + head];
            }
        }
    };
    const uint32_t npairs = (np + 1) >> 1;
    #pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
        if (uint32_t(d) < npairs) {
            load_pair(d, d, true);
            load_pair(d, d, false);
        }
    }
    auto step = [&](int buf, uint32_t pi) {
        const uint32_t i0 = 2 * pi;
        const int n0 = page_tokens(it, i0, last_len);
        const int n1 = page_tokens(it, i0 + 1, last_len);
        f4 sc[1][2];
        const float f0 = a.scale_log2 * ks[buf][0], f1 = a.scale_log2 * ks[buf][1];
        const float v0s = vs[buf][0], v1s = vs[buf][1];
        const bool refill = pi + DEPTH < npairs;
        const bool full = (n0 == kPageSize) && (n1 == kPageSize);
        if constexpr (!PageRaw<D, KVF>::FP8) {
            // 16-bit pages are their own MFMA operands (no copies).  V past
            // a page's valid tokens is zeroed in place (the registers are
            // refilled after the PV products).
            pair_scores<D, F16, 1, 1>(pr[buf][0].k, pr[buf][1].k, qB, sc);
            if (refill) load_pair(buf, pi + DEPTH, true);
            if (!full) {
                mask_v_rows<D>(pr[buf][0].v, g, n0);
                mask_v_rows<D>(pr[buf][1].v, g, n1);
            }
            pair_softmax_pv<D, F16, 1, 1, BLOCK_SCALE>(sc, pr[buf][0].v, pr[buf][1].v, n0, n1, f0, f1, v0s, v1s,
                                                       m, L, O, g);
        } else {
            uint32_t kop[2][KB][4];
            k_operand<D, KVF, F16>(pr[buf][0], kop[0]);
            k_operand<D, KVF, F16>(pr[buf][1], kop[1]);
            pair_scores<D, F16, 1, 1>(kop[0], kop[1], qB, sc);
            if (refill) load_pair(buf, pi + DEPTH, true);
            uint32_t vop[2][4][D / 32];
            if (full) {
                v_operand<D, KVF, F16>(pr[buf][0], g, kPageSize, vop[0]);
                v_operand<D, KVF, F16>(pr[buf][1], g, kPageSize, vop[1]);
            } else {
                v_operand<D, KVF, F16>(pr[buf][0], g, n0, vop[0]);
                v_operand<D, KVF, F16>(pr[buf][1], g, n1, vop[1]);
            }
            pair_softmax_pv<D, F16, 1, 1, BLOCK_SCALE>(sc, vop[0], vop[1], n0, n1, f0, f1, v0s, v1s, m, L, O, g);
        }
        if (refill) load_pair(buf, pi + DEPTH, false);
    };
    for (uint32_t pi = 0; pi < npairs; pi += DEPTH) {
        step(0, pi);
        if (DEPTH == 2 && pi + 1 < npairs) step(DEPTH - 1, pi + 1);
    }
    const float lr[1] = {L[0][0]};
    write_wave_partial<D, 1, true, false>(a, it, 0, 1, dst, m, lr, O, g, c);
}

// ------------------------------------------------------------ group items
// LDS stage of one page pair: planes K(page 0), K(page 1), V(page 0),
// V(page 1), each 16 rows with a 16-byte pad per row (bank spread), then the
// four MX scale records.
template <int D, uint32_t KVF>
struct GroupLayout {
    static constexpr bool FP8 = (KVF == KVF_FP8 || KVF == KVF_MX);
    static constexpr int EB = FP8 ? 1 : 2;
    static constexpr int RB = D * EB;               // row bytes
    static constexpr int RS = RB + 16;              // LDS row stride
    static constexpr int PLANE = kPageSize * RS;
    static constexpr int G = D / 32;
    static constexpr int SREC = kPageSize * G;      // MX scale record bytes
    static constexpr int STAGE = 4 * PLANE + (KVF == KVF_MX ? 4 * SREC : 0);
    static constexpr int CPP = kPageSize * RB / 16; // 16-byte chunks per plane
    static constexpr int NCH = 4 * CPP / (kWaves * 64);   // chunks per thread per pair
    static constexpr int NSC = (KVF == KVF_MX) ? 4 * SREC / 4 : 0;   // scale dwords per pair
    static_assert(NCH >= 1 && (4 * CPP) % (kWaves * 64) == 0, "pair must split evenly");
    static_assert(NSC <= kWaves * 64, "scale records must fit one dword per thread");
};

template <int D, uint32_t KVF>
struct Staged {
    uint32_t d[GroupLayout<D, KVF>::NCH][4];
    uint32_t sc;
};

// Issues the global loads of page pair `pair` of the item into registers.
template <int D, uint32_t KVF>
__device__ __forceinline__ void group_issue(const AttendArgs& a, const Item& it, const uint32_t* ids,
                                            uint32_t pair, Staged<D, KVF>& st, int tid) {
    using L = GroupLayout<D, KVF>;
    const uint32_t np = it.npages;
    const uint32_t i0 = 2 * pair;
    const uint32_t p0 = ids[i0 < np ? i0 : np - 1];
    const uint32_t p1 = ids[i0 + 1 < np ? i0 + 1 : np - 1];
    #pragma unroll
    for (int u = 0; u < L::NCH; ++u) {
        const int q = tid + u * kWaves * 64;
        const int plane = q / L::CPP, within = q - plane * L::CPP;
        const uint32_t page = (plane & 1) ? p1 : p0;
        const uint8_t* src = a.kv + plane_offset(page, plane >> 1, it.kv_head, a.hkv, D, L::EB) + within * 16;
        load_dwords<4>(st.d[u], src);
    }
    if constexpr (KVF == KVF_MX) {
        if (tid < L::NSC) {
            const int rec = tid / (L::SREC / 4), w = tid - rec * (L::SREC / 4);
            const uint32_t page = (rec & 1) ? p1 : p0;
            const uint8_t* src = reinterpret_cast<const uint8_t*>(a.scales) +
                                 ((uint64_t(page) * 2 + (rec >> 1)) * a.hkv + it.kv_head) * L::SREC + 4 * w;
            st.sc = *reinterpret_cast<const uint32_t*>(src);
        }
    }
}

template <int D, uint32_t KVF>
__device__ __forceinline__ void group_commit(uint8_t* stage, const Staged<D, KVF>& st, int tid) {
    using L = GroupLayout<D, KVF>;
    #pragma unroll
    for (int u = 0; u < L::NCH; ++u) {
        const int q = tid + u * kWaves * 64;
        const int plane = q / L::CPP, within = q - plane * L::CPP;
        const int row = within / (L::RB / 16), col = within - row * (L::RB / 16);
        u32x4 v = {st.d[u][0], st.d[u][1], st.d[u][2], st.d[u][3]};
        *reinterpret_cast<u32x4*>(stage + plane * L::PLANE + row * L::RS + col * 16) = v;
    }
    if constexpr (KVF == KVF_MX) {
        if (tid < L::NSC) *reinterpret_cast<uint32_t*>(stage + 4 * L::PLANE + 4 * tid) = st.sc;
    }
}

// Reads one wave's K / V operands of a staged pair from LDS (8-bit codes
// into f16 when H, else bf16).
template <int D, uint32_t KVF, bool H>
__device__ __forceinline__ void group_operands(const uint8_t* stage, int g, int c, int n0, int n1,
                                               uint32_t (&kop)[2][D / 32][4],
                                               uint32_t (&vop)[2][4][D / 32]) {
    using L = GroupLayout<D, KVF>;
    constexpr int KB = D / 32, EPL = D / 16;
    #pragma unroll
    for (int p = 0; p < 2; ++p) {
        const uint8_t* kp = stage + p * L::PLANE + c * L::RS;
        #pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            if constexpr (!L::FP8) {
                load_dwords<4>(kop[p][kb], kp + (kb * 32 + 8 * g) * 2);
            } else {
                uint32_t raw[2];
                load_dwords<2>(raw, kp + kb * 32 + 8 * g);
                float sc = 1.f;
                if constexpr (KVF == KVF_MX) sc = e8m0_to_float(stage[4 * L::PLANE + p * L::SREC + c * L::G + kb]);
                e4m3x4_cvt<H>(raw[0], sc, kop[p][kb][0], kop[p][kb][1]);
                e4m3x4_cvt<H>(raw[1], sc, kop[p][kb][2], kop[p][kb][3]);
            }
        }
    }
    #pragma unroll
    for (int p = 0; p < 2; ++p) {
        const int nt = p ? n1 : n0;
        #pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int tok = 4 * g + j;
            const uint8_t* vp = stage + (2 + p) * L::PLANE + tok * L::RS + c * EPL * L::EB;
            const bool ok = tok < nt;
            if constexpr (!L::FP8) {
                uint32_t raw[EPL / 2];
                load_dwords<EPL / 2>(raw, vp);
                #pragma unroll
                for (int w = 0; w < EPL / 2; ++w) vop[p][j][w] = ok ? raw[w] : 0u;
            } else {
                uint32_t raw[EPL / 4];
                load_dwords<EPL / 4>(raw, vp);
                float sc = 1.f;
                if constexpr (KVF == KVF_MX)
                    sc = e8m0_to_float(stage[4 * L::PLANE + (2 + p) * L::SREC + tok * L::G + (c * EPL) / 32]);
                #pragma unroll
                for (int w = 0; w < EPL / 4; ++w)
                    e4m3x4_cvt<H>(ok ? raw[w] : 0u, sc, vop[p][j][2 * w], vop[p][j][2 * w + 1]);
            }
        }
    }
}

// The group item's pair loop for a wave owning NRT tiles (NRT = 0: the
// wave's rows are all outside the item; it still stages pages and joins
// every barrier).  Two LDS stages; global loads run two pairs ahead in two
// register sets A and B (loop unrolled by two so the sets never move).
template <int D, uint32_t KVF, bool F16, int NRT, int RT>
__device__ __forceinline__ void group_loop(const AttendArgs& a, const Item& it, uint8_t* lds,
                                           const uint32_t* ids, const float* bscale, int tid,
                                           int g, int c, const uint32_t (&qB)[RT][D / 32][4],
                                           float (&m)[RT], f4 (&Lsum)[RT], f4 (&O)[RT][D / 16]) {
    using L = GroupLayout<D, KVF>;
    constexpr bool BLOCK_SCALE = (KVF == KVF_FP8);
    const int last_len = item_last_len(a, it);
    const uint32_t np = it.npages;
    const uint32_t npairs = (np + 1) >> 1;
    uint8_t* stage0 = lds;
    uint8_t* stage1 = lds + L::STAGE;

    auto compute = [&](const uint8_t* stage, uint32_t pair) {
        if constexpr (NRT > 0) {
            const uint32_t i0 = 2 * pair;
            const int n0 = page_tokens(it, i0, last_len);
            const int n1 = page_tokens(it, i0 + 1, last_len);
            float f0 = a.scale_log2, f1 = a.scale_log2, v0s = 1.f, v1s = 1.f;
            if constexpr (BLOCK_SCALE) {
                const uint32_t i1 = i0 + 1 < np ? i0 + 1 : i0;
                f0 *= bscale[2 * i0];
                f1 *= bscale[2 * i1];
                v0s = bscale[2 * i0 + 1];
                v1s = bscale[2 * i1 + 1];
            }
            uint32_t kop[2][D / 32][4];
            uint32_t vop[2][4][D / 32];
            group_operands<D, KVF, F16>(stage, g, c, n0, n1, kop, vop);
            f4 s[RT][2];
            pair_scores<D, F16, NRT, RT>(kop[0], kop[1], qB, s);
            pair_softmax_pv<D, F16, NRT, RT, BLOCK_SCALE>(s, vop[0], vop[1], n0, n1, f0, f1, v0s, v1s, m, Lsum,
                                                          O, g);
        }
    };

    Staged<D, KVF> A, B;
    group_issue<D, KVF>(a, it, ids, 0, A, tid);
    group_issue<D, KVF>(a, it, ids, 1, B, tid);
    group_commit<D, KVF>(stage0, A, tid);
    group_issue<D, KVF>(a, it, ids, 2, A, tid);
    __syncthreads();
    for (uint32_t pi = 0; pi < npairs; pi += 2) {
        compute(stage0, pi);
        group_commit<D, KVF>(stage1, B, tid);      // pair pi+1
        group_issue<D, KVF>(a, it, ids, pi + 3, B, tid);
        __syncthreads();
        if (pi + 1 >= npairs) break;
        compute(stage1, pi + 1);
        group_commit<D, KVF>(stage0, A, tid);      // pair pi+2
        group_issue<D, KVF>(a, it, ids, pi + 4, A, tid);
        __syncthreads();
    }
}

template <int D, uint32_t KVF, bool F16>
__device__ __forceinline__ void group_item(const AttendArgs& a, const Item& it, int tid, int wave, int g,
                                           int c) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * GroupLayout<D, KVF>::STAGE +
                                                        kGroupMaxPages * 4 * (KVF == KVF_FP8 ? 3 : 1)];
    constexpr int RT = kGroupTiles8;
    constexpr int EPL = D / 16;
    constexpr int KB = D / 32;
    // The item's page ids (and FP8 block scales) go to LDS once, so the pair
    // loop reads them without a vector load, whose wait would also drain the
    // page loads running ahead.
    uint32_t* ids = reinterpret_cast<uint32_t*>(lds + 2 * GroupLayout<D, KVF>::STAGE);
    float* bscale = reinterpret_cast<float*>(ids + kGroupMaxPages);
    for (uint32_t i = tid; i < it.npages; i += kWaves * 64) {
        uint32_t pg = a.pages[it.page_off + i];
        pg = pg < a.page_limit ? pg : 0u;
        ids[i] = pg;
        if constexpr (KVF == KVF_FP8) {
            const float* bsc = reinterpret_cast<const float*>(a.scales);
            bscale[2 * i] = bsc[(uint64_t(pg) * 2 + 0) * a.hkv + it.kv_head];
            bscale[2 * i + 1] = bsc[(uint64_t(pg) * 2 + 1) * a.hkv + it.kv_head];
        }
    }
    __syncthreads();
    const uint32_t row0 = uint32_t(wave) * RT * kTileRows;
    const int nrt = it.nrows > row0 ? min(RT, int((it.nrows - row0 + kTileRows - 1) / kTileRows)) : 0;
    uint32_t qB[RT][KB][4];
    uint32_t dst[RT];
    load_q16<D, RT>(a, it, row0, nrt, qB, dst, g, c);
    float m[RT];
    f4 L[RT];
    f4 O[RT][EPL];
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        m[rt] = kNegInf;
        L[rt] = f4{0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int e = 0; e < EPL; ++e) O[rt][e] = f4{0.f, 0.f, 0.f, 0.f};
    }
    if (nrt == RT) group_loop<D, KVF, F16, RT, RT>(a, it, lds, ids, bscale, tid, g, c, qB, m, L, O);
    else if (nrt == 1) group_loop<D, KVF, F16, 1, RT>(a, it, lds, ids, bscale, tid, g, c, qB, m, L, O);
    else group_loop<D, KVF, F16, 0, RT>(a, it, lds, ids, bscale, tid, g, c, qB, m, L, O);
    float lr[RT];
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt) lr[rt] = L[rt][0];
    write_wave_partial<D, RT, true, false>(a, it, row0, nrt, dst, m, lr, O, g, c);
}

// ------------------------------------------------- group items, 16-bit KV
// Pages reach LDS by direct global->LDS loads (global_load_lds_dwordx4, one
// 1 KiB wave load per 64 lanes x 16 bytes): no staging registers and no
// VALU work.  The LDS ring holds NP page pairs; pair p goes to slot p % NP.
// The loads are issued from inline assembly, so the compiler tracks none of
// them and inserts no wait of its own on the ring: before pair p is read
// each wave waits (vmcnt) until its own loads of pair p have landed, and the
// barrier that follows makes every wave's share of the pair visible.  After
// that barrier the slot of pair p - 1 is free and takes pair p + NP - 1.
//
// The item's query rows take the same route: at the start each wave loads
// its rows into the last QSLOTS slots (lane l of a wave load receives bytes
// 16 l.., so each lane reads its own MFMA operand back), then reads them to
// registers; a barrier frees those slots for pages.  The page ids, the row
// targets and the query rows thus cost one dependent memory round trip each
// at the start of an item instead of a chain of them.
//
// A slot holds one page: the K plane (16 rows) then the V plane.  The
// 16-byte chunks of row r are XOR-swizzled (chunk j at position j ^ swz(r)),
// which keeps both read patterns free of bank conflicts:
//   K (A operand of the scores): lane (g, c) reads row c, chunk 4kb + g;
//   V (A operand of O^T, by ds_read_b64_tr_b16): lane (g, c) reads 8 bytes of
//   row 4g + c/4 at dims 16e + 4(c%4); within each 16-lane group the
//   transpose hands lane c the values V[4g + j][16e + c], j = 0..3 — the
//   MFMA's k = 4g + j slots — so the accumulators hold O[row][16e + 4g + i].
// Each wave owns row tiles w, w+4 (RT = 2; one tile for D = 256) of the item.
template <int D>
struct DmaCfg {
    static constexpr int RB = 2 * D;                  // bytes per row
    static constexpr int PLANE = kPageSize * RB;
    static constexpr int PAGE = 2 * PLANE;            // 4, 8 or 16 KiB
    static constexpr int RING = D == 256 ? 128 * 1024 : 64 * 1024;   // LDS bytes of the ring
    static constexpr int NP = RING / (2 * PAGE);      // page pairs in the ring
    static constexpr int DPP = PAGE / (kWaves * 64 * 16);   // wave loads per thread per page
    static constexpr int PER_PAIR = 2 * DPP;          // loads per thread per pair
    static constexpr int RT = group_tiles16(D);       // row tiles per wave
    static constexpr int QBYTES = kWaves * RT * (D / 32) * 1024;   // the item's query rows
    static constexpr int QSLOTS = (QBYTES + 2 * PAGE - 1) / (2 * PAGE);
    static_assert(NP - QSLOTS >= 2, "query rows leave two pair slots");
    static_assert(DPP >= 1 && PLANE % 1024 == 0, "a page must split into 1 KiB wave loads");
    static_assert(NP >= 3 && (NP - 2) * PER_PAIR <= 48, "vmcnt cases");
    static_assert(DPP <= 4, "DmaSrc holds four offsets");
};

// Row swizzle of the 16-byte chunks.  Both read patterns were measured on
// gfx950 (SQ_LDS_BANK_CONFLICT, one probe kernel per pattern): these values
// leave the K reads (ds_read_b128) and the transposed V reads
// (ds_read_b64_tr_b16) without bank conflicts at head_dim 64, 128 and 256.
// Setting bit 0 from row >> 3 as well makes the K reads two-way conflicted.
template <int D>
__device__ __forceinline__ int chunk_swz(int row) {
    if constexpr (D == 64) return ((row >> 1) & 3) << 1;
    else return (row & 7) << 1;
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) void lds_void;

template <bool F16>
__device__ __forceinline__ f4 mma16v(u32x4 a, u32x4 b, f4 c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b),
                                                      c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

// s_waitcnt vmcnt(n) for even n <= 48 (s_waitcnt takes an immediate).
__device__ __forceinline__ void wait_vmcnt(uint32_t n) {
    switch (n) {
        case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
        case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
        case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
        case 6: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
        case 8: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
        case 10: asm volatile("s_waitcnt vmcnt(10)" ::: "memory"); break;
        case 12: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
        case 14: asm volatile("s_waitcnt vmcnt(14)" ::: "memory"); break;
        case 16: asm volatile("s_waitcnt vmcnt(16)" ::: "memory"); break;
        case 18: asm volatile("s_waitcnt vmcnt(18)" ::: "memory"); break;
        case 20: asm volatile("s_waitcnt vmcnt(20)" ::: "memory"); break;
        case 22: asm volatile("s_waitcnt vmcnt(22)" ::: "memory"); break;
        case 24: asm volatile("s_waitcnt vmcnt(24)" ::: "memory"); break;
        case 26: asm volatile("s_waitcnt vmcnt(26)" ::: "memory"); break;
        case 28: asm volatile("s_waitcnt vmcnt(28)" ::: "memory"); break;
        case 30: asm volatile("s_waitcnt vmcnt(30)" ::: "memory"); break;
        case 32: asm volatile("s_waitcnt vmcnt(32)" ::: "memory"); break;
        case 34: asm volatile("s_waitcnt vmcnt(34)" ::: "memory"); break;
        case 36: asm volatile("s_waitcnt vmcnt(36)" ::: "memory"); break;
        case 38: asm volatile("s_waitcnt vmcnt(38)" ::: "memory"); break;
        case 40: asm volatile("s_waitcnt vmcnt(40)" ::: "memory"); break;
        case 42: asm volatile("s_waitcnt vmcnt(42)" ::: "memory"); break;
        case 44: asm volatile("s_waitcnt vmcnt(44)" ::: "memory"); break;
        case 46: asm volatile("s_waitcnt vmcnt(46)" ::: "memory"); break;
        case 48: asm volatile("s_waitcnt vmcnt(48)" ::: "memory"); break;
        default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    }
}

template <int N>
__device__ __forceinline__ void wait_vmcnt_const() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Barrier after this wave's LDS reads have returned (lgkmcnt(0)), so no
// read of a slot can still be in flight when another wave refills it.
__device__ __forceinline__ void block_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);
    compiler_fence();
    __builtin_amdgcn_s_barrier();
    compiler_fence();
}

// Lane byte offsets inside a slot of the K operand read of k-block 0 and
// the transposed V read of d-block 0.  The swizzle is an XOR on the chunk
// index (bits 4..7 of the offset): chunk 4kb + g -> (4kb + g) ^ swz =
// 4 (kb ^ (swz >> 2)) + (g ^ (swz & 3)), so k-block kb is at k ^ (kb << 6)
// and d-block e at v ^ (e << 5) (chunk 2e + h likewise).
struct LdsOffsets {
    uint32_t k;
    uint32_t v;
};

template <int D>
__device__ __forceinline__ LdsOffsets lds_offsets(int g, int c) {
    using C = DmaCfg<D>;
    LdsOffsets o;
    o.k = c * C::RB + ((g ^ chunk_swz<D>(c)) << 4);
    const int row = 4 * g + (c >> 2);
    o.v = C::PLANE + row * C::RB + ((((c & 3) >> 1) ^ chunk_swz<D>(row)) << 4) + ((c & 1) << 3);
    return o;
}

typedef __attribute__((address_space(3))) u32x4 lds_u32x4;

// A lane's LDS read addresses for every k-block and d-block of a pair slot
// at byte offset 0 from `base`.  Bases and slots are multiples of 1 KiB, so
// the swizzle XOR (bits 4..7) and the slot offset commute: the block of a
// slot at offset s is at k[kb] + s, and with s known at compile time the
// read takes it as its immediate offset (no address arithmetic per pair).
template <int D>
struct LdsBases {
    uint32_t k[D / 32];
    uint32_t v[D / 16];
};

template <int D>
__device__ __forceinline__ LdsBases<D> lds_bases(uint32_t base, int g, int c) {
    const LdsOffsets o = lds_offsets<D>(g, c);
    LdsBases<D> b;
    #pragma unroll
    for (int kb = 0; kb < D / 32; ++kb) b.k[kb] = base + (o.k ^ uint32_t(kb << 6));
    #pragma unroll
    for (int e = 0; e < D / 16; ++e) b.v[e] = base + (o.v ^ uint32_t(e << 5));
    return b;
}

// Zeroes the V values of tokens 4g + j >= n (j = 0..3) in one page's half
// (dwords w0, w0+1) of a transposed V operand.
__device__ __forceinline__ void mask_v_tr(u32x4& v, int w0, int g, int n) {
    #pragma unroll
    for (int w = 0; w < 2; ++w) {
        const int t = 4 * g + 2 * w;
        const uint32_t keep = (t < n ? 0x0000FFFFu : 0u) | (t + 1 < n ? 0xFFFF0000u : 0u);
        v[w0 + w] &= keep;
    }
}

// Softmax pieces of the DMA path.  Scores are in log2 units once multiplied
// by f = scale_log2 > 0 (a negative scale is folded into the query's sign).
// A row's reference max m moves only when a score passes it by kLazyDma
// (kLazyDma16 when the probabilities are packed as f16); in between,
// exp2(x - m) stays below 2^32 (bf16 range) or 2^14 (f16, whose range ends
// at 2^16), so the accumulators are not rescaled on the common path.  The check compares the lane's raw score max with
// thr = (m + kLazyDma) / f, kept per row, so the common path spends no
// multiply on it.  The move (always on the item's first pair, where m and
// thr start at -inf) runs on a slow path.
constexpr float kLazyDma = 32.f;
constexpr float kLazyDma16 = 14.f;

template <int RT>
struct RowMax {
    float m[RT];     // reference max, log2 units
    float thr[RT];   // raw score above which m must move
};

// Masks invalid tokens (PARTIAL) and returns the lane's raw score max over
// the pair.
template <int RT, bool PARTIAL>
__device__ __forceinline__ float dma_lane_max(f4 (&s)[RT][2], int rt, int n0, int n1, int g) {
    f4& x0 = s[rt][0];
    f4& x1 = s[rt][1];
    if constexpr (PARTIAL) {
        #pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (4 * g + i >= n0) x0[i] = kNegInf;
            if (4 * g + i >= n1) x1[i] = kNegInf;
        }
    }
    const float a = fmaxf(fmaxf(x0[0], x0[1]), x0[2]);
    const float b = fmaxf(fmaxf(a, x0[3]), x1[0]);
    const float c = fmaxf(fmaxf(b, x1[1]), x1[2]);
    return fmaxf(c, x1[3]);
}

// dma_lane_max for pages whose K scales (ks0, ks1 > 0) are applied to the
// scores rather than to K: the max of raw * ks.
template <int RT, bool PARTIAL>
__device__ __forceinline__ float dma_lane_max_ks(f4 (&s)[RT][2], int rt, int n0, int n1, int g, float ks0,
                                                 float ks1) {
    f4& x0 = s[rt][0];
    f4& x1 = s[rt][1];
    if constexpr (PARTIAL) {
        #pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (4 * g + i >= n0) x0[i] = kNegInf;
            if (4 * g + i >= n1) x1[i] = kNegInf;
        }
    }
    const float r0 = fmaxf(fmaxf(fmaxf(x0[0], x0[1]), x0[2]), x0[3]);
    const float r1 = fmaxf(fmaxf(fmaxf(x1[0], x1[1]), x1[2]), x1[3]);
    return fmaxf(r0 * ks0, r1 * ks1);
}

// The slow path: moves m of every row whose scores passed thr and rescales
// its accumulators.  Rows that did not move get alpha = 1.
template <int D, int NRT, bool F16>
__device__ __forceinline__ void dma_rescale(const float (&lm)[DmaCfg<D>::RT], RowMax<DmaCfg<D>::RT>& rm,
                                         f4 (&Lsum)[DmaCfg<D>::RT], f4 (&O)[DmaCfg<D>::RT][D / 16], float f,
                                         float finv) {
    #pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
        const float mx = rowgroup_max(lm[rt]);
        if (mx > rm.thr[rt]) {
            const float mnew = mx * f;
            const float alpha = rm.m[rt] == kNegInf ? 0.f : fast_exp2(rm.m[rt] - mnew);
            rm.m[rt] = mnew;
            rm.thr[rt] = (mnew + (F16 ? kLazyDma16 : kLazyDma)) * finv;
            Lsum[rt] *= alpha;
            #pragma unroll
            for (int e = 0; e < D / 16; ++e) O[rt][e] *= alpha;
        }
    }
}

// Probabilities of one tile with reference max m (finite: the item's first
// pair always sets it), packed for the PV MFMA, and the row sums they add
// (MFMA against an all-ones operand).
// f0, f1: the two pages' score factors (f times their K scales when those
// are applied to the scores).
template <bool F16>
__device__ __forceinline__ u32x4 dma_probs(const f4 (&x)[2], float f0, float f1, float m, f4& L) {
    const uint32_t one2 = F16 ? 0x3C003C00u : 0x3F803F80u;
    const u32x4 ones = {one2, one2, one2, one2};
    const float nm = -m;
    float p0[4], p1[4];
    #pragma unroll
    for (int i = 0; i < 4; ++i) {
        p0[i] = fast_exp2(__builtin_fmaf(x[0][i], f0, nm));
        p1[i] = fast_exp2(__builtin_fmaf(x[1][i], f1, nm));
    }
    const u32x4 pb = {pack2(p0[0], p0[1], F16), pack2(p0[2], p0[3], F16), pack2(p1[0], p1[1], F16),
                      pack2(p1[2], p1[3], F16)};
    L = mma16v<F16>(ones, pb, L);
    return pb;
}

struct DmaSrc {
    uint32_t loff[4];                 // this lane's source offsets inside a page (DPP <= 4)
    uint64_t page_stride;
};

// One wave load of 64 x 16 bytes from gbase + voff (per lane) to the LDS
// address lds (wave-uniform) + 16 * lane.  Issued from inline assembly: the
// compiler does not track it, so it adds no drain of its own before the LDS
// reads; the pair loop waits for it with explicit vmcnt counts.
__device__ __forceinline__ void dma_x4(uint32_t lds, const void* gbase, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(lds), "v"(voff), "s"(gbase)
                 : "memory", "m0");
}

// Issues this wave's share of the loads of pages pg0, pg1 into pair slot `ps`.
template <int D>
__device__ __forceinline__ void dma_pair_pages(const AttendArgs& a, uint32_t pg0, uint32_t pg1, const DmaSrc& src,
                                               uint32_t ring, uint32_t ps, int wave) {
    using C = DmaCfg<D>;
    #pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint8_t* base = a.kv + uint64_t(q == 0 ? pg0 : pg1) * src.page_stride;
        const uint32_t slot = ring + (2 * ps + q) * C::PAGE + wave * C::DPP * 1024;
        #pragma unroll
        for (int u = 0; u < C::DPP; ++u) dma_x4(slot + u * 1024, base, src.loff[u]);
    }
}

// Issues this wave's share of the loads of pair `pair` into pair slot `ps`.
template <int D>
__device__ __forceinline__ void dma_pair(const AttendArgs& a, const Item& it, const uint32_t* ids,
                                         const DmaSrc& src, uint32_t ring, uint32_t pair, uint32_t ps, int wave) {
    using C = DmaCfg<D>;
    const uint32_t np = it.npages;
    #pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint32_t i = 2 * pair + q < np ? 2 * pair + q : np - 1;
        const uint32_t pg = __builtin_amdgcn_readfirstlane(ids[i]);
        const uint8_t* base = a.kv + uint64_t(pg) * src.page_stride;
        const uint32_t slot = ring + (2 * ps + q) * C::PAGE + wave * C::DPP * 1024;
        #pragma unroll
        for (int u = 0; u < C::DPP; ++u) dma_x4(slot + u * 1024, base, src.loff[u]);
    }
}

// K operands of the page pair in the slot at byte offset s (pages at s and
// s + PAGE from the bases' origin).
template <int D>
__device__ __forceinline__ void dma_k_operands(uint32_t s, const LdsBases<D>& lb, u32x4 (&kop)[2][D / 32]) {
    using C = DmaCfg<D>;
    #pragma unroll
    for (int kb = 0; kb < D / 32; ++kb) {
        kop[0][kb] = *reinterpret_cast<const lds_u32x4*>(uintptr_t(lb.k[kb] + s));
        kop[1][kb] = *reinterpret_cast<const lds_u32x4*>(uintptr_t(lb.k[kb] + s + C::PAGE));
    }
}

// Scores of a page pair for the wave's NRT tiles from its K operands.
template <int D, bool F16, int NRT>
__device__ __forceinline__ void dma_score_mma(const u32x4 (&kop)[2][D / 32],
                                              const u32x4 (&qB)[DmaCfg<D>::RT][D / 32],
                                              f4 (&sc)[DmaCfg<D>::RT][2]) {
    #pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
        sc[rt][0] = f4{0.f, 0.f, 0.f, 0.f};
        sc[rt][1] = f4{0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) {
            sc[rt][0] = mma16v<F16>(kop[0][kb], qB[rt][kb], sc[rt][0]);
            sc[rt][1] = mma16v<F16>(kop[1][kb], qB[rt][kb], sc[rt][1]);
        }
    }
}

// Scores of the page pair in the slot at offset s for the wave's NRT tiles.
template <int D, bool F16, int NRT>
__device__ __forceinline__ void dma_scores(uint32_t s, const LdsBases<D>& lb,
                                           const u32x4 (&qB)[DmaCfg<D>::RT][D / 32],
                                           f4 (&sc)[DmaCfg<D>::RT][2]) {
    u32x4 kop[2][D / 32];
    dma_k_operands<D>(s, lb, kop);
    dma_score_mma<D, F16, NRT>(kop, qB, sc);
}

// The transposed V operands of the page pair in the slot at offset s, all
// d-blocks at once (read before the scores so they land behind the MFMAs).
template <int D>
__device__ __forceinline__ void dma_v_operands(uint32_t s, const LdsBases<D>& lb, u32x4 (&vop)[D / 16]) {
    using C = DmaCfg<D>;
    #pragma unroll
    for (int e = 0; e < D / 16; ++e) {
        const uint32_t ad = lb.v[e] + s;
        const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)uintptr_t(ad));
        const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)uintptr_t(ad + C::PAGE));
        vop[e] = __builtin_shufflevector(__builtin_bit_cast(u32x2, v0), __builtin_bit_cast(u32x2, v1), 0, 1, 2, 3);
    }
}

// Token masks of a page pair: s0[rt] / s1[rt] tokens of the two pages are
// visible to the lane's row of tile rt (scores of the others are masked),
// v0 / v1 tokens hold data (V past them is zeroed, so garbage past a
// sequence's last token cannot reach O through a zero weight).
template <int RT>
struct PairMask {
    int s0[RT], s1[RT];
    int v0, v1;
};

template <int RT>
__device__ __forceinline__ PairMask<RT> uniform_mask(int n0, int n1) {
    PairMask<RT> m;
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        m.s0[rt] = n0;
        m.s1[rt] = n1;
    }
    m.v0 = n0;
    m.v1 = n1;
    return m;
}

// Masks of the pair starting at token t of a causal item: row tile rt sees
// lenr[rt] tokens of the sequence, of which the item holds those below lmax
// (rows of a chunk before the last see past its end: the cap keeps a
// missing second page of the item's last pair masked).
template <int RT>
__device__ __forceinline__ PairMask<RT> causal_mask(int t, const uint32_t (&lenr)[RT], int lmax) {
    auto cl = [](int x) { return min(max(x, 0), kPageSize); };
    PairMask<RT> m;
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int len = min(int(lenr[rt]), lmax);
        m.s0[rt] = cl(len - t);
        m.s1[rt] = cl(len - t - kPageSize);
    }
    m.v0 = cl(lmax - t);
    m.v1 = cl(lmax - t - kPageSize);
    return m;
}

// One step of the pair loop after its barrier: the lazy-max check of pair
// p (scores already in sc) and its rare rescale, then the LDS reads (V of
// pair p from the slot at offset vs and, when NEXT, K of pair p + 1 from the
// slot at ks), the score MFMAs of pair p + 1 interleaved with the softmax of
// pair p, and the PV MFMAs.  PART masks tokens past n0 / n1 (the item's
// last pair only); the last pair has no next pair (NEXT false).  KS: the
// pages' K scales ks0, ks1 multiply the scores (K was staged unscaled).
template <int D, bool F16, int NRT, bool PART, bool NEXT, bool KS = false, bool PF16 = F16>
__device__ __forceinline__ void dma_step(uint32_t vs, uint32_t ks, const PairMask<DmaCfg<D>::RT>& pm,
                                         const LdsBases<D>& lb,
                                         const u32x4 (&qB)[DmaCfg<D>::RT][D / 32], f4 (&sc)[DmaCfg<D>::RT][2],
                                         u32x4 (&vop)[D / 16], RowMax<DmaCfg<D>::RT>& rm,
                                         f4 (&Lsum)[DmaCfg<D>::RT], f4 (&O)[DmaCfg<D>::RT][D / 16], int g,
                                         float f, float finv, float ks0 = 1.f, float ks1 = 1.f) {
    constexpr int RT = DmaCfg<D>::RT, KB = D / 32;
    bool need = false;
    float lm[RT];
    #pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
        if constexpr (KS) lm[rt] = dma_lane_max_ks<RT, PART>(sc, rt, pm.s0[rt], pm.s1[rt], g, ks0, ks1);
        else lm[rt] = dma_lane_max<RT, PART>(sc, rt, pm.s0[rt], pm.s1[rt], g);
        need |= lm[rt] > rm.thr[rt];
    }
    if (__ballot(need)) dma_rescale<D, NRT, PF16>(lm, rm, Lsum, O, f, finv);
    // Branch-free from here, so the scheduler sees one region, in this
    // order (pinned: a wave issues in order, and at most 15 LDS reads may
    // be outstanding before issue stalls): the K reads of pair p + 1; the
    // softmax of pair p (VALU), which needs no LDS, while they are in
    // flight; the score MFMAs of pair p + 1 with the V reads of pair p
    // issued one between each two; then the PV MFMAs of pair p.
    __builtin_amdgcn_sched_barrier(0);
    u32x4 kop[2][KB];
    if constexpr (NEXT) dma_k_operands<D>(ks, lb, kop);
    __builtin_amdgcn_sched_barrier(0);
    u32x4 pB[RT];
    const float f0 = KS ? f * ks0 : f, f1 = KS ? f * ks1 : f;
    #pragma unroll
    for (int rt = 0; rt < NRT; ++rt) pB[rt] = dma_probs<PF16>(sc[rt], f0, f1, rm.m[rt], Lsum[rt]);
    __builtin_amdgcn_sched_barrier(0);
    dma_v_operands<D>(vs, lb, vop);
    if constexpr (NEXT) {
        dma_score_mma<D, F16, NRT>(kop, qB, sc);
        constexpr int NM = NRT * 2 * KB, NV = D / 8;   // score MFMAs, V reads
        #pragma unroll
        for (int k = 0; k < (NM > NV ? NM : NV); ++k) {
            if (k < NV) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // one LDS read
            if (k < NM) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (PART) {
        #pragma unroll
        for (int e = 0; e < D / 16; ++e) {
            mask_v_tr(vop[e], 0, g, pm.v0);
            mask_v_tr(vop[e], 2, g, pm.v1);
        }
    }
    #pragma unroll
    for (int e = 0; e < D / 16; ++e) {
        #pragma unroll
        for (int rt = 0; rt < NRT; ++rt) O[rt][e] = mma16v<PF16>(vop[e], pB[rt], O[rt][e]);
    }
}

// Compile-time loop index.
template <int J>
struct Idx {
    static constexpr int value = J;
};

template <int J, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (J < N) {
        f(Idx<J>{});
        static_for<J + 1, N>(f);
    }
}

// Where the rows of a wave's tiles come from and go to: the byte offset of
// the query row in q and the partial-state row, read once per item.  Rows
// past the item's last are given its last row (their query is zeroed and
// nothing is written for them).
template <int RT>
struct RowTargets {
    uint32_t qoff[RT];
    uint32_t dst[RT];
    uint32_t len[RT];    // tokens the row sees (causal items only)
};

template <int D, int RT>
__device__ __forceinline__ void dma_row_targets(const AttendArgs& a, const Item& it, int wave, int c,
                                                RowTargets<RT>& rtg) {
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        uint32_t row = uint32_t(rt * kWaves + wave) * kTileRows + c;
        row = row < it.nrows ? row : it.nrows - 1;
        uint32_t seq, slot, qh;
        row_target(a, it, row, seq, slot, qh);
        rtg.qoff[rt] = (seq * a.hq + qh) * uint32_t(D * 2);
        rtg.dst[rt] = slot * a.hq + qh;
        rtg.len[rt] = (it.flags & kItemCausal) ? a.row_len[seq] : 0u;
    }
}

template <int D, bool F16, int NRT, bool TAIL, bool CAUSAL>
__device__ __forceinline__ void dma_group_loop(const AttendArgs& a, const Item& it, const uint32_t* ids,
                                               uint8_t* ring, int tid, int wave, int g, int c,
                                               const RowTargets<DmaCfg<D>::RT>& rtg, int last_len,
                                               const ItemLim& lim,
                                               u32x4 (&qB)[DmaCfg<D>::RT][D / 32],
                                               RowMax<DmaCfg<D>::RT>& rm, f4 (&Lsum)[DmaCfg<D>::RT],
                                               f4 (&O)[DmaCfg<D>::RT][D / 16]) {
    using C = DmaCfg<D>;
    constexpr uint32_t P = C::NP, QS = C::QSLOTS;
    constexpr int KB = D / 32;
    const uint32_t np = it.npages;
    const uint32_t npairs = (np + 1) >> 1;
    DmaSrc src;
    src.page_stride = uint64_t(2) * a.hkv * C::PLANE;
    #pragma unroll
    for (int u = 0; u < C::DPP; ++u) {
        const int b = (wave * C::DPP + u) * 1024 + 16 * (tid & 63);
        const int plane = b / C::PLANE, rem = b - plane * C::PLANE;
        const int row = rem / C::RB, pos = (rem - row * C::RB) >> 4;
        const int j = pos ^ chunk_swz<D>(row);
        src.loff[u] = uint32_t((plane * a.hkv + it.kv_head) * C::PLANE + row * C::RB + j * 16);
    }
    const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(uint32_t(reinterpret_cast<uintptr_t>(ring)));
    const LdsBases<D> lb = lds_bases<D>(ring_lds, g, c);
    const float f = a.scale_log2;   // > 0 (a negative scale is in q_sign)
    const float finv = 1.f / f;
    const uint32_t qsign = a.q_sign;
    // Every load the compiler issued (row targets, page ids) has landed
    // before the ring loads start, so no compiler-inserted wait can drain
    // the ring.
    __builtin_amdgcn_s_waitcnt(0x0070);
    compiler_fence();
    // Query rows into the last QS slots, the first pairs into the others.
    const uint32_t q_lds = ring_lds + (P - QS) * 2 * C::PAGE + wave * (C::RT * KB * 1024);
    #pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
        #pragma unroll
        for (int kb = 0; kb < KB; ++kb)
            dma_x4(q_lds + (rt * KB + kb) * 1024, static_cast<const uint8_t*>(a.q), rtg.qoff[rt] + kb * 64 + 16 * g);
    }
    const uint32_t pro = min(P - QS, npairs);
    #pragma unroll 1
    for (uint32_t q = 0; q < pro; ++q) dma_pair<D>(a, it, ids, src, ring_lds, q, q, wave);
    wait_vmcnt(pro * C::PER_PAIR);   // loads land in issue order: the query rows are in
    if constexpr (NRT > 0) {
        const uint8_t* qw = ring + (P - QS) * 2 * C::PAGE + wave * (C::RT * KB * 1024) + 16 * (tid & 63);
        #pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
            const bool valid = uint32_t(rt * kWaves + wave) * kTileRows + c < it.nrows;
            #pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                const u32x4 v = *reinterpret_cast<const u32x4*>(qw + (rt * KB + kb) * 1024) ^ qsign;
                qB[rt][kb] = valid ? v : u32x4{0u, 0u, 0u, 0u};
            }
        }
    }
    block_barrier();   // every wave holds its query rows: their slots take pages
    #pragma unroll 1
    for (uint32_t q = pro; q < min(P - 1, npairs); ++q) dma_pair<D>(a, it, ids, src, ring_lds, q, q, wave);
    // Software pipeline: step pi computes the scores of pair pi + 1 while
    // it finishes pair pi.  It reads K of pair pi + 1 and V of pair pi;
    // after its barrier the slot of pair pi - 1 is free and takes pair
    // pi + P - 1.  Pair p sits in slot p % P, so the steps are unrolled
    // over the P slots and every LDS read takes its slot as an immediate
    // offset.  Issued before step pi: pairs < min(pi + P - 1, npairs).
    // Order inside a step (pinned with scheduling barriers, since a wave
    // issues in order): the row-max check of pair pi (its scores are
    // already in registers) and the rare rescale; then all LDS reads; then
    // the probabilities of pair pi (VALU) interleaved with the score MFMAs
    // of pair pi + 1; then the PV MFMAs of pair pi.  The last pair runs
    // apart: it may hold partial pages and has no next pair to score.
    constexpr int RT = C::RT;
    constexpr uint32_t SLOT = 2 * C::PAGE;
    f4 sc[RT][2];
    u32x4 vop[D / 16];
    wait_vmcnt((min(P - 1, npairs) - 1) * C::PER_PAIR);   // pair 0 has landed
    block_barrier();
    if constexpr (NRT > 0) dma_scores<D, F16, NRT>(0, lb, qB, sc);
    // Page ids of the pair the next refill loads (pair pi + P - 1), read from
    // LDS a step ahead so the refill does not wait on them.
    uint32_t nid0 = ids[min(2 * (P - 1), np - 1)];
    uint32_t nid1 = ids[min(2 * (P - 1) + 1, np - 1)];
    const uint32_t nmain = npairs - 1;
    #pragma unroll 1
    for (uint32_t p0 = 0; p0 < nmain; p0 += P) {
        static_for<0, int(P)>([&](auto J) {
            constexpr uint32_t j = decltype(J)::value;
            const uint32_t pi = p0 + j;
            if (pi >= nmain) return;
            if (pi + P - 1 <= npairs) wait_vmcnt_const<(P - 3) * C::PER_PAIR>();   // pair pi + 1 has landed
            else wait_vmcnt((npairs - pi - 2) * C::PER_PAIR);
            block_barrier();
            if (pi + P - 1 < npairs)
                dma_pair_pages<D>(a, __builtin_amdgcn_readfirstlane(nid0), __builtin_amdgcn_readfirstlane(nid1),
                                  src, ring_lds, (j + P - 1) % P, wave);
            nid0 = ids[min(2 * (pi + P), np - 1)];
            nid1 = ids[min(2 * (pi + P) + 1, np - 1)];
            if constexpr (NRT > 0) {
                // A causal item's pairs below every row's last token need no
                // mask; the ones crossing the diagonal mask per row.
                const int t = CAUSAL ? int(lim.tok0 + 2 * kPageSize * pi) : 0;
                if (CAUSAL && t + 2 * kPageSize > int(lim.lmin))
                    dma_step<D, F16, NRT, true, true>(j * SLOT, ((j + 1) % P) * SLOT,
                                                      causal_mask<RT>(t, rtg.len, int(lim.lmax)), lb, qB, sc,
                                                      vop, rm, Lsum, O, g, f, finv);
                else
                    dma_step<D, F16, NRT, false, true>(j * SLOT, ((j + 1) % P) * SLOT,
                                                       uniform_mask<RT>(kPageSize, kPageSize), lb, qB, sc, vop,
                                                       rm, Lsum, O, g, f, finv);
            }
        });
    }
    // The last pair: its loads were waited for (vmcnt(0)) and made visible
    // by the previous step's barrier (or the prologue's); it refills nothing
    // and reads no K, so it needs no barrier of its own.
    if constexpr (NRT > 0) {
        const uint32_t pl = nmain;
        PairMask<RT> pm;
        if constexpr (CAUSAL) {
            pm = causal_mask<RT>(int(lim.tok0 + 2 * kPageSize * pl), rtg.len, int(lim.lmax));
        } else {
            const int n0 = TAIL && 2 * pl + 1 == np ? last_len : kPageSize;
            const int n1 = 2 * pl + 1 >= np ? 0 : (TAIL && 2 * pl + 2 == np ? last_len : kPageSize);
            pm = uniform_mask<RT>(n0, n1);
        }
        dma_step<D, F16, NRT, true, false>((pl % P) * SLOT, 0, pm, lb, qB, sc, vop, rm, Lsum, O, g, f, finv);
    }
}

// Query rows of a wave's tiles in a DMA group item: tile rt of wave w covers
// rows (rt * kWaves + w) * 16 .. +16.
template <int D, int RT, bool PF>
__device__ __forceinline__ void write_partial_dma(const AttendArgs& a, const Item& it, int wave, int nrt,
                                                  const RowTargets<RT>& rtg, const float (&m)[RT],
                                                  const f4 (&L)[RT], const f4 (&O)[RT][D / 16], int g, int c,
                                                  bool f16) {
    constexpr int EPL = D / 16;
    const uint32_t (&dst)[RT] = rtg.dst;
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        if (rt >= nrt) break;
        const uint32_t row = uint32_t(rt * kWaves + wave) * kTileRows + c;
        const float lt = L[rt][0];
        const float inv = lt > 0.f ? 1.f / lt : 0.f;
        if (PF && a.out_direct) {   // the row's only partial state is its output
            if (row < it.nrows) {
                uint8_t* o = static_cast<uint8_t*>(a.out_direct) + rtg.qoff[rt];
                #pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    const f4 v = O[rt][e] * inv;
                    *reinterpret_cast<u32x2*>(o + 2 * (16 * e + 4 * g)) =
                        u32x2{pack2(v[0], v[1], f16), pack2(v[2], v[3], f16)};
                }
            }
            continue;
        }
        float mx = 0.f;
        #pragma unroll
        for (int e = 0; e < EPL; ++e)
            #pragma unroll
            for (int i = 0; i < 4; ++i) mx = fmaxf(mx, fabsf(O[rt][e][i]));
        const int k = partial_exp(rowgroup_max(mx) * inv);
        const float sc = __builtin_amdgcn_ldexpf(inv, -k);
        if (row < it.nrows) {
            uint16_t* o = static_cast<uint16_t*>(a.ws_o) + uint64_t(dst[rt]) * D;
            #pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const f4 v = O[rt][e] * sc;
                *reinterpret_cast<u32x2*>(o + 16 * e + 4 * g) = u32x2{pack2(v[0], v[1], true), pack2(v[2], v[3], true)};
            }
            if (g == 0) a.ws_lse[dst[rt]] = PartialLse{lt > 0.f ? m[rt] + log2f(lt) : kNegInf, float(k)};
        }
    }
}

template <int D, bool F16, int NRT, bool PF>
__device__ __forceinline__ void dma_group_run(const AttendArgs& a, const Item& it, const uint32_t* ids,
                                              uint8_t* ring, int tid, int wave, int g, int c,
                                              const RowTargets<DmaCfg<D>::RT>& rtg, int last_len) {
    using C = DmaCfg<D>;
    constexpr int RT = C::RT, EPL = D / 16, KB = D / 32;
    u32x4 qB[RT][KB];
    RowMax<RT> rm;
    f4 L[RT];
    f4 O[RT][EPL];
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        rm.m[rt] = kNegInf;
        rm.thr[rt] = kNegInf;
        L[rt] = f4{0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int e = 0; e < EPL; ++e) O[rt][e] = f4{0.f, 0.f, 0.f, 0.f};
    }
    if constexpr (PF) {   // prefill plans: every item is causal
        const ItemLim lim = a.item_lim[blockIdx.x];
        dma_group_loop<D, F16, NRT, false, true>(a, it, ids, ring, tid, wave, g, c, rtg, last_len, lim, qB, rm, L,
                                                 O);
    } else if (it.flags & kItemTail) {
        dma_group_loop<D, F16, NRT, true, false>(a, it, ids, ring, tid, wave, g, c, rtg, last_len, ItemLim{},
                                                 qB, rm, L, O);
    } else {
        dma_group_loop<D, F16, NRT, false, false>(a, it, ids, ring, tid, wave, g, c, rtg, last_len, ItemLim{},
                                                  qB, rm, L, O);
    }
    write_partial_dma<D, RT, PF>(a, it, wave, NRT, rtg, rm.m, L, O, g, c, F16);
}

// Item fields as wave-uniform values (they are: the item is the workgroup's),
// so loop bounds and page addressing stay in scalar registers.
__device__ __forceinline__ Item uniform_item(const Item& it) {
    Item u;
    u.page_off = __builtin_amdgcn_readfirstlane(it.page_off);
    u.npages = __builtin_amdgcn_readfirstlane(it.npages);
    u.seq_off = __builtin_amdgcn_readfirstlane(it.seq_off);
    u.row_begin = __builtin_amdgcn_readfirstlane(it.row_begin);
    u.nrows = __builtin_amdgcn_readfirstlane(it.nrows);
    u.kv_head = __builtin_amdgcn_readfirstlane(it.kv_head);
    u.flags = __builtin_amdgcn_readfirstlane(it.flags);
    u.tail_seq = __builtin_amdgcn_readfirstlane(it.tail_seq);
    return u;
}

template <int D, bool F16, bool PF>
__device__ __forceinline__ void group_item_dma(const AttendArgs& a, const Item& item, int tid, int wave, int g,
                                               int c) {
    using C = DmaCfg<D>;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[C::RING];
    __shared__ uint32_t ids[PF ? kPrefillMaxPages : kGroupMaxPages];
    const Item it = uniform_item(item);
    // Row targets, the last page's length and the page ids load together.
    RowTargets<C::RT> rtg;
    dma_row_targets<D, C::RT>(a, it, wave, c, rtg);
    const int last_len = item_last_len(a, it);
    for (uint32_t i = tid; i < it.npages; i += kWaves * 64) {
        const uint32_t pg = a.pages[it.page_off + i];
        ids[i] = pg < a.page_limit ? pg : 0u;
    }
    __syncthreads();
    // Tiles of this wave that hold rows: tiles w, w+4, ... below ceil(nrows/16).
    const int ntiles = int((it.nrows + kTileRows - 1) / kTileRows);
    const int nrt = ntiles > wave ? min(C::RT, (ntiles - wave + kWaves - 1) / kWaves) : 0;
    if (nrt >= 3) dma_group_run<D, F16, C::RT, PF>(a, it, ids, ring, tid, wave, g, c, rtg, last_len);
    else if (nrt == 2) dma_group_run<D, F16, 2, PF>(a, it, ids, ring, tid, wave, g, c, rtg, last_len);
    else if (nrt == 1) dma_group_run<D, F16, 1, PF>(a, it, ids, ring, tid, wave, g, c, rtg, last_len);
    else dma_group_run<D, F16, 0, PF>(a, it, ids, ring, tid, wave, g, c, rtg, last_len);
}

// ------------------------------------------- group items, FP8 / MXFP8 KV
// Raw E4M3 pages and their scales reach LDS by direct loads into a ring of
// NPR raw pairs.  Each raw pair is then converted by the whole workgroup
// into a bf16 pair slot laid out as the 16-bit path's (swizzled rows), and
// the 16-bit pair loop's compute (dma_step) runs on those slots.  MXFP8
// elements take their E8M0 group scale in the exact power-of-two conversion;
// with an E4M3 block scale, K codes are converted exactly (the scale then
// multiplies the scores, so a large attention scale cannot amplify a
// rounding of code * scale) and V is converted exactly to f32, multiplied
// by its scale and rounded once to bf16.  Per iteration pi: wait for raw pair
// pi + 1, barrier, refill the raw slot of pair pi - 1 (converted two
// iterations ago), convert raw pair pi + 1 into bf16 slot (pi + 1) & 1,
// barrier, compute.  Head_dim 128 and 256 (64 keeps the register path).
template <int D>
struct Dma8Cfg {
    using C16 = DmaCfg<D>;
    static constexpr int RAW_PLANE = kPageSize * D;              // E4M3 bytes of one plane
    static constexpr int RAW_PAGE = 2 * RAW_PLANE;
    static constexpr int RAW_PAIR = 2 * RAW_PAGE;
    static constexpr int NPR = 4;                                // raw ring pairs
    static constexpr int RDPP = RAW_PAGE / (kWaves * 1024);      // wave loads per thread per raw page
    static constexpr int PER_PAIR = 2 * RDPP + 1;                // + the pair's scale load
    static constexpr int SCALES = 1024;                          // LDS bytes of one raw pair's scales
    static constexpr int SREC = kPageSize * (D / 32);            // MXFP8 scale bytes of one plane
    static constexpr int NCH = 4 * SREC / 16;                    // 16-byte chunks of a pair's MX scales
    static constexpr int BF_PAIR = 2 * C16::PAGE;                // bf16 pair slot
    static constexpr int RAW_BYTES = NPR * (RAW_PAIR + SCALES);
    static constexpr int LDS = RAW_BYTES + 2 * BF_PAIR;
    static constexpr int CONV = RAW_PAIR / (kWaves * 64 * 32);   // 32-element runs per thread per pair
    static_assert(RDPP >= 1 && RDPP <= 4 && CONV >= 1, "head_dim 128 or 256");
    static_assert(C16::QBYTES <= 2 * BF_PAIR, "query rows fit the bf16 slots");
    static_assert(4 * SREC <= SCALES && NCH <= 64, "scale slot");
    static_assert(NPR * PER_PAIR <= 63, "vmcnt range");
};

// One wave load of 64 x 4 bytes from gbase + voff (per lane) to lds + 4 * lane.
__device__ __forceinline__ void dma_x1(uint32_t lds, const void* gbase, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2"
                 :
                 : "s"(lds), "v"(voff), "s"(gbase)
                 : "memory", "m0");
}

// s_waitcnt vmcnt(n), n <= 63, from a run-time value.
__device__ __forceinline__ void wait_vmcnt_any(uint32_t n) {
#define DH_VMCNT_CASE(k) case k: asm volatile("s_waitcnt vmcnt(" #k ")" ::: "memory"); break;
    switch (n) {
        DH_VMCNT_CASE(0) DH_VMCNT_CASE(1) DH_VMCNT_CASE(2) DH_VMCNT_CASE(3) DH_VMCNT_CASE(4)
        DH_VMCNT_CASE(5) DH_VMCNT_CASE(6) DH_VMCNT_CASE(7) DH_VMCNT_CASE(8) DH_VMCNT_CASE(9)
        DH_VMCNT_CASE(10) DH_VMCNT_CASE(11) DH_VMCNT_CASE(12) DH_VMCNT_CASE(13) DH_VMCNT_CASE(14)
        DH_VMCNT_CASE(15) DH_VMCNT_CASE(16) DH_VMCNT_CASE(17) DH_VMCNT_CASE(18) DH_VMCNT_CASE(19)
        DH_VMCNT_CASE(20) DH_VMCNT_CASE(21) DH_VMCNT_CASE(22) DH_VMCNT_CASE(23) DH_VMCNT_CASE(24)
        DH_VMCNT_CASE(25) DH_VMCNT_CASE(26) DH_VMCNT_CASE(27) DH_VMCNT_CASE(28) DH_VMCNT_CASE(29)
        DH_VMCNT_CASE(30) DH_VMCNT_CASE(31) DH_VMCNT_CASE(32) DH_VMCNT_CASE(33) DH_VMCNT_CASE(34)
        DH_VMCNT_CASE(35) DH_VMCNT_CASE(36) DH_VMCNT_CASE(37) DH_VMCNT_CASE(38) DH_VMCNT_CASE(39)
        DH_VMCNT_CASE(40) DH_VMCNT_CASE(41) DH_VMCNT_CASE(42) DH_VMCNT_CASE(43) DH_VMCNT_CASE(44)
        DH_VMCNT_CASE(45) DH_VMCNT_CASE(46) DH_VMCNT_CASE(47) DH_VMCNT_CASE(48)
        default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    }
#undef DH_VMCNT_CASE
}

// Source offsets (per lane) of one raw pair's loads.
template <int D>
struct Dma8Src {
    uint32_t loff[Dma8Cfg<D>::RDPP];    // inside a raw page, this wave's share
    uint64_t page_stride;
    uint32_t s_rel;                     // scale load: offset inside the (page, plane) record
    uint32_t s_plane;                   // scale load: plane of this lane's chunk
    bool s_page1;                       // scale load: this lane's chunk belongs to the pair's second page
};

template <int D, uint32_t KVF>
__device__ __forceinline__ Dma8Src<D> dma8_src(const AttendArgs& a, const Item& it, int wave, int lane) {
    using C8 = Dma8Cfg<D>;
    Dma8Src<D> s;
    s.page_stride = uint64_t(2) * a.hkv * C8::RAW_PLANE;
    #pragma unroll
    for (int u = 0; u < C8::RDPP; ++u) {
        const int b = (wave * C8::RDPP + u) * 1024 + 16 * lane;
        const int plane = b / C8::RAW_PLANE, rem = b - plane * C8::RAW_PLANE;
        s.loff[u] = uint32_t((plane * a.hkv + it.kv_head) * C8::RAW_PLANE + rem);
    }
    if constexpr (KVF == KVF_MX) {
        const int k = lane % C8::NCH, pp = k / (C8::SREC / 16);
        s.s_page1 = (pp >> 1) != 0;
        s.s_plane = uint32_t(pp & 1);
        s.s_rel = uint32_t((k % (C8::SREC / 16)) * 16);
    } else {
        const int e = lane & 3;
        s.s_page1 = (e >> 1) != 0;
        s.s_plane = uint32_t(e & 1);
        s.s_rel = 0;
    }
    return s;
}

// Issues this wave's loads of pages pg0, pg1 (and their scales) into raw slot rs.
template <int D, uint32_t KVF>
__device__ __forceinline__ void dma8_pair(const AttendArgs& a, const Item& it, uint32_t pg0, uint32_t pg1,
                                          const Dma8Src<D>& src, uint32_t raw_lds, uint32_t rs, int wave) {
    using C8 = Dma8Cfg<D>;
    const uint32_t slot = raw_lds + rs * (C8::RAW_PAIR + C8::SCALES);
    #pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint8_t* base = a.kv + uint64_t(q == 0 ? pg0 : pg1) * src.page_stride;
        const uint32_t dst = slot + q * C8::RAW_PAGE + wave * C8::RDPP * 1024;
        #pragma unroll
        for (int u = 0; u < C8::RDPP; ++u) dma_x4(dst + u * 1024, base, src.loff[u]);
    }
    const uint32_t pg = src.s_page1 ? pg1 : pg0;
    const uint32_t rec = (pg * 2 + src.s_plane) * a.hkv + it.kv_head;
    if constexpr (KVF == KVF_MX)
        dma_x4(slot + C8::RAW_PAIR, a.scales, rec * uint32_t(C8::SREC) + src.s_rel);
    else
        dma_x1(slot + C8::RAW_PAIR, a.scales, rec * 4u);
}

// Converts raw slot rs into bf16 slot bs (the whole workgroup; tid < 256).
template <int D, uint32_t KVF, bool HK, bool HV>
__device__ __forceinline__ void dma8_convert(uint8_t* ring, uint32_t rs, uint32_t bs, int tid) {
    using C8 = Dma8Cfg<D>;
    using C = DmaCfg<D>;
    const uint8_t* raw = ring + rs * (C8::RAW_PAIR + C8::SCALES);
    const uint8_t* scl = raw + C8::RAW_PAIR;
    uint8_t* bf = ring + C8::RAW_BYTES + bs * C8::BF_PAIR;
    #pragma unroll
    for (int k = 0; k < C8::CONV; ++k) {
        const int o = 32 * (tid + kWaves * 64 * k);
        const int page = o / C8::RAW_PAGE, po = o - page * C8::RAW_PAGE;
        const int plane = po / C8::RAW_PLANE, pr = po - plane * C8::RAW_PLANE;
        const int row = pr / D, col0 = pr - row * D;
        const u32x4 w0 = *reinterpret_cast<const u32x4*>(raw + o);
        const u32x4 w1 = *reinterpret_cast<const u32x4*>(raw + o + 16);
        const uint32_t wd[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
        uint32_t out[16];
        if constexpr (KVF == KVF_MX) {
            const float sc = e8m0_to_float(scl[(page * 2 + plane) * C8::SREC + row * (D / 32) + col0 / 32]);
            if (plane == 0) {
                #pragma unroll
                for (int w = 0; w < 8; ++w) e4m3x4_cvt<HK>(wd[w], sc, out[2 * w], out[2 * w + 1]);
            } else {
                #pragma unroll
                for (int w = 0; w < 8; ++w) e4m3x4_cvt<HV>(wd[w], sc, out[2 * w], out[2 * w + 1]);
            }
        } else if (plane == 0) {
            // K: the codes alone (exact in bf16); the block scale multiplies
            // the scores, so the attention scale does not amplify a rounding
            // of code * scale.  (plane is wave-uniform: a wave converts 2048
            // consecutive bytes, whole planes at head_dim 128 and 256.)
            #pragma unroll
            for (int w = 0; w < 8; ++w) e4m3x4_cvt<HK>(wd[w], 1.f, out[2 * w], out[2 * w + 1]);
        } else {
            // V: code * scale in f32, rounded once to bf16 or f16 (RNE).
            const float sc = *reinterpret_cast<const float*>(scl + 4 * (page * 2 + plane));
            #pragma unroll
            for (int w = 0; w < 8; ++w) {
                const f2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(wd[w], false);
                const f2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(wd[w], true);
                out[2 * w] = pack2(lo[0] * sc, lo[1] * sc, HV);
                out[2 * w + 1] = pack2(hi[0] * sc, hi[1] * sc, HV);
            }
        }
        uint8_t* rowp = bf + page * C::PAGE + plane * C::PLANE + row * C::RB;
        #pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int pos = (col0 / 8 + j) ^ chunk_swz<D>(row);
            *reinterpret_cast<u32x4*>(rowp + pos * 16) = u32x4{out[4 * j], out[4 * j + 1], out[4 * j + 2], out[4 * j + 3]};
        }
    }
}

template <int D, uint32_t KVF, bool F16, int NRT, bool TAIL, bool CAUSAL, bool PF16 = F16>
__device__ __forceinline__ void dma8_group_loop(const AttendArgs& a, const Item& it, const uint32_t* ids,
                                                uint8_t* ring, int tid, int wave, int g, int c,
                                                const RowTargets<DmaCfg<D>::RT>& rtg, int last_len,
                                                const ItemLim& lim,
                                                u32x4 (&qB)[DmaCfg<D>::RT][D / 32],
                                                RowMax<DmaCfg<D>::RT>& rm, f4 (&Lsum)[DmaCfg<D>::RT],
                                                f4 (&O)[DmaCfg<D>::RT][D / 16]) {
    using C = DmaCfg<D>;
    using C8 = Dma8Cfg<D>;
    constexpr uint32_t P = C8::NPR;
    constexpr int RT = C::RT, KB = D / 32;
    const uint32_t np = it.npages;
    const uint32_t npairs = (np + 1) >> 1;
    const int lane = tid & 63;
    const Dma8Src<D> src = dma8_src<D, KVF>(a, it, wave, lane);
    const uint32_t raw_lds = __builtin_amdgcn_readfirstlane(uint32_t(reinterpret_cast<uintptr_t>(ring)));
    const uint32_t bf_lds = raw_lds + C8::RAW_BYTES;
    const LdsBases<D> lb = lds_bases<D>(bf_lds, g, c);
    const float f = a.scale_log2;   // > 0 (a negative scale is in q_sign)
    const float finv = 1.f / f;
    const uint32_t qsign = a.q_sign;
    // FP8 block scale: K is staged unscaled and the pages' K scales (in the
    // raw slot of the pair being finished, records [page][K|V]) multiply
    // the scores.
    constexpr bool KS = KVF == KVF_FP8;
    auto k_scales = [&](uint32_t rs, float& k0, float& k1) {
        const float* sk = reinterpret_cast<const float*>(ring + rs * (C8::RAW_PAIR + C8::SCALES) + C8::RAW_PAIR);
        k0 = sk[0];
        k1 = sk[2];
    };
    auto page_id = [&](uint32_t i) { return __builtin_amdgcn_readfirstlane(ids[i < np ? i : np - 1]); };
    // Every compiler-issued load (row targets, page ids) has landed before
    // the ring loads start, so no compiler-inserted wait drains the ring.
    __builtin_amdgcn_s_waitcnt(0x0070);
    compiler_fence();
    const uint32_t q_lds = bf_lds + wave * (RT * KB * 1024);
    #pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
        #pragma unroll
        for (int kb = 0; kb < KB; ++kb)
            dma_x4(q_lds + (rt * KB + kb) * 1024, static_cast<const uint8_t*>(a.q), rtg.qoff[rt] + kb * 64 + 16 * g);
    }
    const uint32_t pro = min(P - 1, npairs);
    #pragma unroll 1
    for (uint32_t q = 0; q < pro; ++q) dma8_pair<D, KVF>(a, it, page_id(2 * q), page_id(2 * q + 1), src, raw_lds, q, wave);
    wait_vmcnt_any(pro * C8::PER_PAIR);   // loads land in issue order: the query rows are in
    if constexpr (NRT > 0) {
        const uint8_t* qw = ring + C8::RAW_BYTES + wave * (RT * KB * 1024) + 16 * lane;
        #pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
            const bool valid = uint32_t(rt * kWaves + wave) * kTileRows + c < it.nrows;
            #pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                const u32x4 v = *reinterpret_cast<const u32x4*>(qw + (rt * KB + kb) * 1024) ^ qsign;
                qB[rt][kb] = valid ? v : u32x4{0u, 0u, 0u, 0u};
            }
        }
    }
    wait_vmcnt_any((pro - 1) * C8::PER_PAIR);   // raw pair 0 has landed
    block_barrier();                             // query rows read; raw pair 0 visible
    dma8_convert<D, KVF, F16, PF16>(ring, 0, 0, tid);
    block_barrier();
    f4 sc[RT][2];
    u32x4 vop[D / 16];
    if constexpr (NRT > 0) dma_scores<D, F16, NRT>(0, lb, qB, sc);
    uint32_t ps = 0, psn = 1;   // raw slots of pairs pi, pi + 1
    uint32_t nid0 = page_id(2 * (P - 1)), nid1 = page_id(2 * (P - 1) + 1);
    // Step pi: raw pair pi + 1 is converted into bf16 slot (pi + 1) & 1 while
    // pair pi is finished from slot pi & 1; steps are unrolled by two so the
    // bf16 slots are immediate offsets.  The last pair runs apart (partial
    // pages, nothing to score next, nothing to convert).
    const uint32_t nmain = npairs - 1;
    #pragma unroll 1
    for (uint32_t p0 = 0; p0 < nmain; p0 += 2) {
        static_for<0, 2>([&](auto J) {
            constexpr uint32_t j = decltype(J)::value;
            const uint32_t pi = p0 + j;
            if (pi >= nmain) return;
            // raw pair pi + 1 has landed: an immediate count while pairs
            // are still being issued (a runtime count is a tree of branches)
            if (pi + P - 1 <= npairs) wait_vmcnt_const<(P - 3) * C8::PER_PAIR>();
            else wait_vmcnt_any((npairs - pi - 2) * C8::PER_PAIR);
            block_barrier();
            if (pi + P - 1 < npairs) dma8_pair<D, KVF>(a, it, nid0, nid1, src, raw_lds, ps == 0 ? P - 1 : ps - 1, wave);
            nid0 = page_id(2 * (pi + P));
            nid1 = page_id(2 * (pi + P) + 1);
            dma8_convert<D, KVF, F16, PF16>(ring, psn, (j + 1) & 1, tid);
            block_barrier();
            if constexpr (NRT > 0) {
                float ks0 = 1.f, ks1 = 1.f;
                if constexpr (KS) k_scales(ps, ks0, ks1);
                const int t = CAUSAL ? int(lim.tok0 + 2 * kPageSize * pi) : 0;
                if (CAUSAL && t + 2 * kPageSize > int(lim.lmin))
                    dma_step<D, F16, NRT, true, true, KS, PF16>(j * C8::BF_PAIR, ((j + 1) & 1) * C8::BF_PAIR,
                                                                  causal_mask<RT>(t, rtg.len, int(lim.lmax)), lb, qB,
                                                                  sc, vop, rm, Lsum, O, g, f, finv, ks0, ks1);
                else
                    dma_step<D, F16, NRT, false, true, KS, PF16>(j * C8::BF_PAIR, ((j + 1) & 1) * C8::BF_PAIR,
                                                                   uniform_mask<RT>(kPageSize, kPageSize), lb, qB,
                                                                   sc, vop, rm, Lsum, O, g, f, finv, ks0, ks1);
            }
            ps = psn;
            psn = psn + 1 == P ? 0 : psn + 1;
        });
    }
    // The last pair was converted and made visible by the previous step (or
    // the prologue); every raw load has landed (the last wait was vmcnt(0)).
    if constexpr (NRT > 0) {
        const uint32_t pl = nmain;
        PairMask<RT> pm;
        if constexpr (CAUSAL) {
            pm = causal_mask<RT>(int(lim.tok0 + 2 * kPageSize * pl), rtg.len, int(lim.lmax));
        } else {
            const int n0 = TAIL && 2 * pl + 1 == np ? last_len : kPageSize;
            const int n1 = 2 * pl + 1 >= np ? 0 : (TAIL && 2 * pl + 2 == np ? last_len : kPageSize);
            pm = uniform_mask<RT>(n0, n1);
        }
        float ks0 = 1.f, ks1 = 1.f;
        if constexpr (KS) k_scales(ps, ks0, ks1);
        dma_step<D, F16, NRT, true, false, KS, PF16>((pl & 1) * C8::BF_PAIR, 0, pm, lb, qB, sc, vop, rm, Lsum, O,
                                                      g, f, finv, ks0, ks1);
    }
}

template <int D, uint32_t KVF, bool F16, int NRT, bool PF, bool PF16 = F16>
__device__ __forceinline__ void dma8_group_run(const AttendArgs& a, const Item& it, const uint32_t* ids,
                                               uint8_t* ring, int tid, int wave, int g, int c,
                                               const RowTargets<DmaCfg<D>::RT>& rtg, int last_len) {
    using C = DmaCfg<D>;
    constexpr int RT = C::RT, EPL = D / 16, KB = D / 32;
    u32x4 qB[RT][KB];
    RowMax<RT> rm;
    f4 L[RT];
    f4 O[RT][EPL];
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        rm.m[rt] = kNegInf;
        rm.thr[rt] = kNegInf;
        L[rt] = f4{0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int e = 0; e < EPL; ++e) O[rt][e] = f4{0.f, 0.f, 0.f, 0.f};
    }
    if constexpr (PF) {   // prefill plans: every item is causal
        const ItemLim lim = a.item_lim[blockIdx.x];
        dma8_group_loop<D, KVF, F16, NRT, false, true, PF16>(a, it, ids, ring, tid, wave, g, c, rtg, last_len, lim, qB, rm,
                                                  L, O);
    } else if (it.flags & kItemTail) {
        dma8_group_loop<D, KVF, F16, NRT, true, false, PF16>(a, it, ids, ring, tid, wave, g, c, rtg, last_len, ItemLim{},
                                                  qB, rm, L, O);
    } else {
        dma8_group_loop<D, KVF, F16, NRT, false, false, PF16>(a, it, ids, ring, tid, wave, g, c, rtg, last_len, ItemLim{},
                                                   qB, rm, L, O);
    }
    write_partial_dma<D, RT, PF>(a, it, wave, NRT, rtg, rm.m, L, O, g, c, F16);
}

// Whether the V values of KV head h in page `page` fit f16: FP8's
// per-(page, head) scale at most 146 (448 x 146 < 65504), MXFP8's E8M0
// exponents of the page's 16 tokens x D/32 groups at most 134 (448 x 2^7).
// Smaller values only lose bits below f16's least subnormal, far under the
// output tolerance.
template <int D, uint32_t KVF>
__device__ __forceinline__ bool v_fits_f16(const AttendArgs& a, uint32_t page, uint32_t h) {
    const uint8_t* sc = static_cast<const uint8_t*>(a.scales);
    if constexpr (KVF == KVF_FP8) {
        const uint64_t rec = uint64_t(2) * a.hkv * 4;
        const float s = *reinterpret_cast<const float*>(sc + page * rec + (a.hkv + h) * 4);
        return s <= 146.f;   // NaN: false
    } else {
        constexpr int G = D / 32;
        const uint64_t rec = uint64_t(2) * a.hkv * kPageSize * G;
        const u32x4* p = reinterpret_cast<const u32x4*>(sc + page * rec + uint64_t(a.hkv + h) * kPageSize * G);
        uint32_t big = 0;
        #pragma unroll
        for (int j = 0; j < G; ++j) {
            const u32x4 w = p[j];
            #pragma unroll
            for (int i = 0; i < 4; ++i)
                #pragma unroll
                for (int b = 0; b < 32; b += 8) big |= ((w[i] >> b) & 0xFFu) > 134u ? 1u : 0u;
        }
        return big == 0;
    }
}

// 8-bit group item.  With bf16 queries the probabilities and V go into
// the PV products as f16 when every V value of the item's pages fits f16
// (checked on the scales with the page ids): bf16's 8-bit significand on
// the probabilities was the largest error term at C5's shape (1.2e-2 beyond
// the output rounding in an emulation of this arithmetic, 4e-3 with f16
// probabilities in the shared-prefix items).  The scores stay bf16 x bf16.
template <int D, uint32_t KVF, bool F16, bool PF>
__device__ __forceinline__ void group_item_dma8(const AttendArgs& a, const Item& item, int tid, int wave, int g,
                                                int c) {
    using C = DmaCfg<D>;
    using C8 = Dma8Cfg<D>;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[C8::LDS];
    __shared__ uint32_t ids[PF ? kPrefillMaxPages : kGroupMaxPages];
    constexpr bool V16 = !F16 && !PF;   // probabilities may go f16
    const Item it = uniform_item(item);
    RowTargets<C::RT> rtg;
    dma_row_targets<D, C::RT>(a, it, wave, c, rtg);
    const int last_len = item_last_len(a, it);
    int big = 0;
    for (uint32_t i = tid; i < it.npages; i += kWaves * 64) {
        const uint32_t pg = a.pages[it.page_off + i];
        const uint32_t id = pg < a.page_limit ? pg : 0u;
        ids[i] = id;
        if constexpr (V16) big |= v_fits_f16<D, KVF>(a, id, it.kv_head) ? 0 : 1;
    }
    bool pf16 = false;
    if constexpr (V16) pf16 = __syncthreads_or(big) == 0;
    else __syncthreads();
    const int ntiles = int((it.nrows + kTileRows - 1) / kTileRows);
    const int nrt = ntiles > wave ? min(C::RT, (ntiles - wave + kWaves - 1) / kWaves) : 0;
    auto run = [&](auto pfI) {
        constexpr bool P16 = decltype(pfI)::value != 0;
        if (nrt >= 2) dma8_group_run<D, KVF, F16, C::RT, PF, P16>(a, it, ids, ring, tid, wave, g, c, rtg, last_len);
        else if (nrt == 1) dma8_group_run<D, KVF, F16, 1, PF, P16>(a, it, ids, ring, tid, wave, g, c, rtg, last_len);
        else dma8_group_run<D, KVF, F16, 0, PF, P16>(a, it, ids, ring, tid, wave, g, c, rtg, last_len);
    };
    if constexpr (V16) {
        if (pf16) run(Idx<1>{});
        else run(Idx<0>{});
    } else {
        run(Idx<F16 ? 1 : 0>{});
    }
}

// ---------------------------------------------------------------- attend16
// q in bf16 (KV bf16 / FP8 E4M3 / MXFP8) or f16 (KV f16); bf16/f16 MFMA.
// Partial-row layout seen by the merge: a lane loads 16 bytes of a state row.
template <int D, uint32_t OUT>
struct MergeShape {
    static constexpr int ES = OUT == 2 ? 4 : 2;      // bytes per partial element (f32 or scaled f16)
    static constexpr int EPL = 16 / ES;              // elements per lane per load
    static constexpr int LPS = D / EPL;              // lanes per state row
    static constexpr int SPI = 64 / LPS;             // states per load instruction
    static constexpr int MAX_NV = 64 / SPI < 16 ? 64 / SPI : 16;
    static_assert(LPS >= 1 && LPS <= 64 && 64 % LPS == 0, "head_dim");
    // loads per pass for rows of at most `states` states (a power of two)
    static constexpr int nv_for(int states) {
        int need = (states + SPI - 1) / SPI, nv = 1;
        while (nv < need && nv < MAX_NV) nv *= 2;
        return nv;
    }
};

template <int D, uint32_t OUT, int NV>
__device__ __forceinline__ void merge_row(const void* ws_o, const PartialLse* ws_lse, void* out, uint32_t hq,
                                          uint32_t b, uint32_t qh, uint32_t s0, uint32_t n, int lane);

// Direct decode plans: after its waves wrote their partial states, the
// workgroup merges its rows (one (sequence, KV head, row block): the rows of
// its first item) over the sequence's slots and writes out.  The states are
// read back through the cache right after they were written: a workgroup
// fence and barrier order the writes of every wave before the reads.
template <int D, uint32_t OUT>
__device__ __forceinline__ void wave_task_merge(const AttendArgs& a, int wave, int lane) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    const Item it = uniform_item(a.items[a.n_group_items + (blockIdx.x - a.n_group_items) * kWaves]);
    for (uint32_t row = uint32_t(wave); row < it.nrows; row += kWaves) {
        uint32_t seq, slot, qh;
        row_target(a, it, row, seq, slot, qh);
        seq = __builtin_amdgcn_readfirstlane(seq);
        qh = __builtin_amdgcn_readfirstlane(qh);
        const uint32_t s0 = __builtin_amdgcn_readfirstlane(a.slot_ptr[seq]);
        const uint32_t n = __builtin_amdgcn_readfirstlane(a.slot_ptr[seq + 1]) - s0;
        // at most kWaves states per row
        merge_row<D, OUT, MergeShape<D, OUT>::nv_for(kWaves)>(a.ws_o, a.ws_lse, a.out, a.hq, seq, qh, s0, n, lane);
    }
}

template <int D, uint32_t KVF, bool F16>
__global__ __launch_bounds__(256, D >= 256 ? 1 : 2) void attend16_kernel(AttendArgs a) {
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
    // Wave index as a wave-uniform (scalar) value: page-list reads then go
    // through the scalar cache and never wait on the vector loads in flight.
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t ng = group_item_count(a);
    if (blockIdx.x < ng) {
        const Item it = a.items[blockIdx.x];
        if constexpr ((KVF == KVF_FP8 || KVF == KVF_MX) && D == 64) group_item<D, KVF, F16>(a, it, tid, wave, g, c);
        else if constexpr (KVF == KVF_FP8 || KVF == KVF_MX) group_item_dma8<D, KVF, F16, false>(a, it, tid, wave, g, c);
        else group_item_dma<D, F16, false>(a, it, tid, wave, g, c);
    } else {
        const uint32_t idx = wave_item_index(a, wave, ng);
        if (idx < wave_item_end(a)) {
            const Item it = a.csr_hdr ? csr_wave_item(a, idx, ng) : a.items[idx];
            if (it.npages) wave_item<D, KVF, F16>(a, it, g, c);   // direct tasks pad with empty items
        }
        if (a.wave_direct) wave_task_merge<D, F16 ? 0u : 1u>(a, wave, tid & 63);
    }
}

// Prefill plans: causal group items only (every workgroup one item); the
// 16-bit and FP8 / MXFP8 direct-load paths at head_dim 128 and 256 and the
// 16-bit one at 64.  A kernel of its own, so the per-row token masks do not
// add to the decode kernel's registers.
template <int D, uint32_t KVF, bool F16>
__global__ __launch_bounds__(256, D >= 256 ? 1 : 2) void prefill16_kernel(AttendArgs a) {
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    if (blockIdx.x >= a.n_group_items) return;
    const Item it = a.items[blockIdx.x];
    if constexpr (KVF == KVF_FP8 || KVF == KVF_MX) group_item_dma8<D, KVF, F16, true>(a, it, tid, wave, g, c);
    else group_item_dma<D, F16, true>(a, it, tid, wave, g, c);
}

// ---------------------------------------------------------------- attend32
// f32 q and f32 KV (wave items only): v_mfma_f32_16x16x4_f32, one page per
// step, 16 rows per wave.
//   S^T: A = K[token c][g*D/4 + kb], B = Q[row c][g*D/4 + kb], kb < D/4.
//   O^T: for token group i: A = V[4g+i][c*EPL + e], B = P[row c][4g+i].
// One wave item of attend32_kernel.
template <int D>
__device__ __forceinline__ void attend32_item(const AttendArgs& a, const Item& it, int lane, int g, int c) {
    constexpr int KQ = D / 4;
    constexpr int EPL = D / 16;

    float qv[KQ];
    uint32_t dst[1] = {0u};
    if (uint32_t(c) < it.nrows) {
        uint32_t seq, slot, qh;
        row_target(a, it, c, seq, slot, qh);
        dst[0] = slot * a.hq + qh;
        const float* qp = reinterpret_cast<const float*>(a.q) + (uint64_t(seq) * a.hq + qh) * D + g * KQ;
        load_dwords<KQ>(reinterpret_cast<uint32_t*>(qv), qp);
        #pragma unroll
        for (int k = 0; k < KQ; ++k) qv[k] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, qv[k]) ^ a.q_sign);
    } else {
        #pragma unroll
        for (int k = 0; k < KQ; ++k) qv[k] = 0.f;
    }

    float m[1] = {kNegInf}, l[1] = {0.f};
    f4 O[1][EPL];
    #pragma unroll
    for (int e = 0; e < EPL; ++e) O[0][e] = f4{0.f, 0.f, 0.f, 0.f};

    const int last_len = item_last_len(a, it);
    const uint32_t* pages = a.pages + it.page_off;
    const uint32_t np = it.npages;
    const uint64_t plane_bytes = uint64_t(kPageSize) * D * 4;

    // DEPTH pages in flight: buffer p % DEPTH holds page p; once page p is
    // consumed its registers take page p + DEPTH.  Two at head_dim 64 (32
    // registers a page); one above (64 or 128), where a second page would
    // cost occupancy.
    constexpr int DEPTH = D <= 64 ? 2 : 1;
    float kb[DEPTH][KQ];
    float vb[DEPTH][4][EPL];
    bool bad = false;
    auto load = [&](int buf, uint32_t pi) {
        const uint32_t pg = pages[pi];
        bad |= pg >= a.page_limit;
        const uint8_t* kp = a.kv + plane_offset(pg < a.page_limit ? pg : 0u, 0, it.kv_head, a.hkv, D, 4);
        const uint8_t* vp = kp + uint64_t(a.hkv) * plane_bytes;
        load_dwords<KQ>(reinterpret_cast<uint32_t*>(kb[buf]), kp + (c * D + g * KQ) * 4);
        #pragma unroll
        for (int i = 0; i < 4; ++i)
            load_dwords<EPL>(reinterpret_cast<uint32_t*>(vb[buf][i]), vp + ((4 * g + i) * D + c * EPL) * 4);
    };
    #pragma unroll
    for (int d = 0; d < DEPTH; ++d)
        if (uint32_t(d) < np) load(d, d);
    #pragma unroll 1
    for (uint32_t p0 = 0; p0 < np; p0 += DEPTH) {
        static_for<0, DEPTH>([&](auto J) {
            constexpr int j = decltype(J)::value;
            const uint32_t pi = p0 + j;
            if (pi >= np) return;
            const int n0 = page_tokens(it, pi, last_len);
            f4 s = {0.f, 0.f, 0.f, 0.f};
            #pragma unroll
            for (int k = 0; k < KQ; ++k) s = __builtin_amdgcn_mfma_f32_16x16x4f32(kb[j][k], qv[k], s, 0, 0, 0);
            float x[4];
            float mx = kNegInf;
            #pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[i] = (4 * g + i < n0) ? s[i] * a.scale_log2 : kNegInf;
                mx = fmaxf(mx, x[i]);
            }
            mx = rowgroup_max(mx);
            const float mnew = fmaxf(m[0], mx);
            const float muse = (mnew == kNegInf) ? 0.f : mnew;
            const float alpha = fast_exp2(m[0] - muse);
            m[0] = mnew;
            float ps = 0.f;
            #pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[i] = fast_exp2(x[i] - muse);
                ps += x[i];
            }
            l[0] = l[0] * alpha + ps;
            #pragma unroll
            for (int e = 0; e < EPL; ++e) O[0][e] *= alpha;
            #pragma unroll
            for (int i = 0; i < 4; ++i) {
                // V past the page's valid tokens: zero (its weight is zero,
                // garbage there must not reach O).
                const bool ok = 4 * g + i < n0;
                #pragma unroll
                for (int e = 0; e < EPL; ++e)
                    O[0][e] = __builtin_amdgcn_mfma_f32_16x16x4f32(ok ? vb[j][i][e] : 0.f, x[i], O[0][e], 0, 0, 0);
            }
            if (pi + DEPTH < np) load(j, pi + DEPTH);
        });
    }
    if (__ballot(bad) && a.seq_bad && lane == 0) a.seq_bad[it.tail_seq] = 1u;
    write_wave_partial<D, 1, false, true>(a, it, 0, 1, dst, m, l, O, g, c);
}

template <int D>
__global__ __launch_bounds__(256) void attend32_kernel(AttendArgs a) {
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t idx = wave_item_index(a, wave, group_item_count(a));   // f32: no group items
    if (idx < wave_item_end(a)) {
        const Item it = a.csr_hdr ? csr_wave_item(a, idx, 0) : a.items[idx];
        if (it.npages) attend32_item<D>(a, it, lane, g, c);   // direct tasks pad with empty items
    }
    if (a.wave_direct) wave_task_merge<D, 2u>(a, wave, lane);
}

// ------------------------------------------------------------------ merge
// One wave per (sequence, query head): log-sum-exp over the sequence's
// partial states; no partial state -> zeros (backend.rs:218-222).
// Lane l reads the log-sum-exp of slots l, l+64, ...; the wave reduces their
// max and weights with cross-lane operations, then accumulates the slots'
// O rows sixteen at a time so sixteen loads are in flight per lane instead of
// one dependent load per slot.
__device__ __forceinline__ float wave_max(float x) {
    #pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
    return x;
}

__device__ __forceinline__ float wave_sum(float x) {
    #pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}

// PL consecutive partial-O elements starting at element e of the partial
// rows: fp32 when the output is f32 (OUT == 2), else scaled f16.
template <int OUT, int PL>
__device__ __forceinline__ void load_partial(const void* ws, uint64_t e, float (&v)[PL]) {
    if constexpr (OUT == 2) {
        const float* o = static_cast<const float*>(ws) + e;
        #pragma unroll
        for (int q = 0; q < PL; ++q) v[q] = o[q];
    } else if constexpr (PL == 1) {
        v[0] = float(static_cast<const _Float16*>(ws)[e]);
    } else {
        const uint32_t* o = reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(ws) + e);
        uint32_t w[PL / 2];
        #pragma unroll
        for (int q = 0; q < PL / 2; ++q) w[q] = o[q];
        #pragma unroll
        for (int q = 0; q < PL / 2; ++q) {
            v[2 * q] = unpack_lo(w[q], true);
            v[2 * q + 1] = unpack_hi(w[q], true);
        }
    }
}

// merge_row for at most 64 states: a lane loads 16 bytes of one state row
// (LPS lanes cover a row, so one load instruction reads SPI = 64 / LPS
// states), all of a pass's loads are issued together with the
// log-sum-exps, and the SPI lane groups' weighted sums are added across
// lanes at the end.  One pass covers NV * SPI states (NV chosen for the
// plan's most states per row), so such a row costs one memory round trip
// after its slot range.
template <int D, uint32_t OUT, int NV>
__device__ __forceinline__ void merge_row_v(const void* ws_o, const PartialLse* ws_lse, void* out, uint32_t hq,
                                            uint32_t b, uint32_t qh, uint32_t s0, uint32_t n, int lane) {
    using MS = MergeShape<D, OUT>;
    constexpr int ES = MS::ES, EPL = MS::EPL, LPS = MS::LPS, SPI = MS::SPI;
    static_assert(NV >= 1 && NV <= MS::MAX_NV, "loads per pass");
    const int grp = lane / LPS, e = lane % LPS;
    float acc[EPL];
    #pragma unroll
    for (int i = 0; i < EPL; ++i) acc[i] = 0.f;
    float W = 0.f;
    if (n != 0) {
        const PartialLse pk = uint32_t(lane) < n ? ws_lse[uint64_t(s0 + lane) * hq + qh]
                                                 : PartialLse{kNegInf, 0.f};
        const uint8_t* base = static_cast<const uint8_t*>(ws_o) + (uint64_t(s0) * hq + qh) * (D * ES) + 16 * e;
        const uint64_t sstride = uint64_t(hq) * (D * ES);
        u32x4 v[NV];
        auto load = [&](uint32_t j0) {
            #pragma unroll
            for (int u = 0; u < NV; ++u) {
                const uint32_t st = min(j0 + uint32_t(u * SPI + grp), n - 1);
                v[u] = *reinterpret_cast<const u32x4*>(base + st * sstride);
            }
        };
        load(0);
        const float M = wave_max(pk.lse);
        if (M != kNegInf) {
            const float wk = pk.lse == kNegInf ? 0.f : fast_exp2(pk.lse - M);
            W = wk;
            const float wo = __builtin_amdgcn_ldexpf(wk, int(pk.k));   // weight of the stored (scaled) O
            for (uint32_t j0 = 0; j0 < n; j0 += NV * SPI) {
                if (j0) load(j0);
                #pragma unroll
                for (int u = 0; u < NV; ++u) {
                    const uint32_t st = j0 + uint32_t(u * SPI + grp);
                    const float w = __shfl(wo, int(st & 63u), 64);
                    const float wu = st < n ? w : 0.f;
                    if constexpr (OUT == 2) {
                        #pragma unroll
                        for (int i = 0; i < 4; ++i) acc[i] += wu * __uint_as_float(v[u][i]);
                    } else {
                        #pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            acc[2 * i] += wu * unpack_lo(v[u][i], true);
                            acc[2 * i + 1] += wu * unpack_hi(v[u][i], true);
                        }
                    }
                }
            }
        }
    }
    #pragma unroll
    for (int o = LPS; o < 64; o <<= 1)
        #pragma unroll
        for (int i = 0; i < EPL; ++i) acc[i] += __shfl_xor(acc[i], o, 64);
    W = wave_sum(W);
    const float inv = W > 0.f ? 1.f / W : 0.f;
    if (lane < LPS) {
        uint8_t* o = static_cast<uint8_t*>(out) + ((uint64_t(b) * hq + qh) * D + e * EPL) * (OUT == 2 ? 4 : 2);
        if constexpr (OUT == 2) {
            *reinterpret_cast<f4*>(o) = f4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
        } else {
            u32x4 w;
            #pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = pack2(acc[2 * i] * inv, acc[2 * i + 1] * inv, OUT == 0);
            *reinterpret_cast<u32x4*>(o) = w;
        }
    }
}

// One wave merges output row (b, qh) over partial slots s0 .. s0 + n - 1
// (no slot: zeros).  NV > 0: rows of up to 64 states take merge_row_v.
// Otherwise (NV = 0, and rows of more than 64 states) a lane loads 4-8 bytes
// of every state row, U partial rows per pass (32 for NV = 0, else 16): a
// row of at most U states costs one round trip after its slot range.  On
// MI355X the vector form is faster for 36 states at head_dim 64 (C2, one
// pass instead of two: 10.5 -> 9.6 us a step), the same for 2-9 (C1, C4,
// C5), and slower for 19 at head_dim 128 (C3: 28.0 against 27.6), which
// keeps the scalar form.
template <int D, uint32_t OUT, int NV>
__device__ __forceinline__ void merge_row(const void* ws_o, const PartialLse* ws_lse, void* out, uint32_t hq,
                                          uint32_t b, uint32_t qh, uint32_t s0, uint32_t n, int lane) {
    if constexpr (NV > 0) {
        if (n <= 64) {
            merge_row_v<D, OUT, NV>(ws_o, ws_lse, out, hq, b, qh, s0, n, lane);
            return;
        }
    }
    if constexpr (NV < 0) {   // loads per pass from the row's own state count (wave-uniform)
        using MS = MergeShape<D, OUT>;
        constexpr int S = MS::SPI, MX = MS::MAX_NV;
        if (n <= uint32_t(S)) {
            merge_row_v<D, OUT, 1>(ws_o, ws_lse, out, hq, b, qh, s0, n, lane);
            return;
        }
        if (n <= uint32_t(4 * S)) {
            merge_row_v<D, OUT, (MX < 4 ? MX : 4)>(ws_o, ws_lse, out, hq, b, qh, s0, n, lane);
            return;
        }
        if (n <= 64) {
            merge_row_v<D, OUT, MX>(ws_o, ws_lse, out, hq, b, qh, s0, n, lane);
            return;
        }
    }
    constexpr int U = NV == 0 ? 32 : 16;
    constexpr int PL = D / 64;
    float acc[PL];
    #pragma unroll
    for (int k = 0; k < PL; ++k) acc[k] = 0.f;
    float W = 0.f;
    if (n != 0 && n <= 64) {
        // One pass: the log-sum-exps and the first U partial rows are loaded
        // together (neither depends on the other), so a row with up to U
        // partial states costs one memory round trip after slot_ptr.
        const PartialLse pk = uint32_t(lane) < n ? ws_lse[uint64_t(s0 + lane) * hq + qh]
                                                 : PartialLse{kNegInf, 0.f};
        float v[U][PL];
        #pragma unroll
        for (int u = 0; u < U; ++u)
            load_partial<OUT, PL>(ws_o, (uint64_t(s0 + min(uint32_t(u), n - 1)) * hq + qh) * D + lane * PL, v[u]);
        const float M = wave_max(pk.lse);
        if (M != kNegInf) {
            const float wk = pk.lse == kNegInf ? 0.f : fast_exp2(pk.lse - M);
            W = wk;
            const float wo = __builtin_amdgcn_ldexpf(wk, int(pk.k));   // weight of the stored (scaled) O
            for (uint32_t j0 = 0; j0 < n; j0 += U) {
                if (j0) {
                    #pragma unroll
                    for (int u = 0; u < U; ++u)
                        load_partial<OUT, PL>(ws_o, (uint64_t(s0 + min(j0 + u, n - 1)) * hq + qh) * D + lane * PL,
                                              v[u]);
                }
                #pragma unroll
                for (int u = 0; u < U; ++u) {
                    const float w = (j0 + u < n) ? __shfl(wo, int(j0 + u), 64) : 0.f;
                    #pragma unroll
                    for (int q = 0; q < PL; ++q) acc[q] += w * v[u][q];
                }
            }
        }
    } else if (n > 64) {
        float M = kNegInf;
        for (uint32_t k = lane; k < n; k += 64) M = fmaxf(M, ws_lse[uint64_t(s0 + k) * hq + qh].lse);
        M = wave_max(M);
        if (M != kNegInf) {
            for (uint32_t base = 0; base < n; base += 64) {
                // Weight of slot base + lane, then the slots' O rows in groups of U.
                const uint32_t k = base + lane;
                const PartialLse pk = k < n ? ws_lse[uint64_t(s0 + k) * hq + qh] : PartialLse{kNegInf, 0.f};
                const float wk = pk.lse == kNegInf ? 0.f : fast_exp2(pk.lse - M);
                W += wk;
                const float wo = __builtin_amdgcn_ldexpf(wk, int(pk.k));   // weight of the stored (scaled) O
                const uint32_t cnt = min(64u, n - base);
                for (uint32_t j0 = 0; j0 < cnt; j0 += U) {
                    float v[U][PL];
                    #pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const uint32_t j = min(j0 + u, cnt - 1);
                        load_partial<OUT, PL>(ws_o, (uint64_t(s0 + base + j) * hq + qh) * D + lane * PL, v[u]);
                    }
                    #pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const float w = (j0 + u < cnt) ? __shfl(wo, int(j0 + u), 64) : 0.f;
                        #pragma unroll
                        for (int q = 0; q < PL; ++q) acc[q] += w * v[u][q];
                    }
                }
            }
        }
    }
    W = wave_sum(W);
    const float inv = W > 0.f ? 1.f / W : 0.f;
    const uint64_t ob = (uint64_t(b) * hq + qh) * D + lane * PL;
    #pragma unroll
    for (int k = 0; k < PL; ++k) {
        const float v = acc[k] * inv;
        if constexpr (OUT == 2) reinterpret_cast<float*>(out)[ob + k] = v;
        else if constexpr (OUT == 1) reinterpret_cast<__bf16*>(out)[ob + k] = (__bf16)v;
        else reinterpret_cast<_Float16*>(out)[ob + k] = (_Float16)v;
    }
}

template <int D, uint32_t OUT, int NV>
__global__ __launch_bounds__(256) void merge_kernel(MergeArgs a) {
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (a.status && blockIdx.x == 0 && threadIdx.x < 64) {   // the CSR call's status
        uint32_t bad = 0;
        for (uint32_t b = lane; b < a.batch; b += 64) bad |= a.seq_bad[b];
        const bool any = __ballot(bad != 0) != 0;
        if (lane == 0) *a.status = a.csr_hdr->overflow ? 2 : (any ? 1 : 0);   // DH_ENOMEM / DH_EINVAL / DH_OK
    }
    if (row >= a.batch * a.hq) return;
    const uint32_t b = row / a.hq, qh = row - b * a.hq;
    // Plans whose sequences all have n slots: the slot range is b*n .. +n,
    // one dependent load fewer before the partial states.
    const uint32_t s0 = a.uniform_slots ? b * a.uniform_slots : a.slot_ptr[b];
    const uint32_t n = a.uniform_slots ? a.uniform_slots
                                       : ((a.seq_bad && a.seq_bad[b]) ? 0u : a.slot_ptr[b + 1] - s0);
    merge_row<D, OUT, NV>(a.ws_o, a.ws_lse, a.out, a.hq, b, qh, s0, n, lane);
}

// ------------------------------------------------- decode from device CSR
// The CSR planning kernel runs as one workgroup of NT threads: one wave for
// batches of at most 64 sequences (one sequence a lane, no barriers between
// its passes), one wave per SIMD (256 threads) beyond.  Each thread keeps
// the page counts of its first csr_reg_seqs(NT) sequences in registers
// across the passes (the small variant's code stays short: it runs on a CU
// whose instruction cache has not seen it).
constexpr uint32_t kCsrSmallThreads = 64, kCsrThreads = 256;
constexpr uint32_t csr_reg_seqs(uint32_t nt) { return nt == kCsrSmallThreads ? 1u : 2u; }

// Inclusive scan over the wave (lane i: the sum, or minimum, of lanes
// 0..i): row shifts by 1, 2, 4, 8 within each 16-lane row, then the last
// lane of row 0 / 2 into rows 1 / 3 (row_bcast:15) and of row 1 into rows
// 2 and 3 (row_bcast:31).  A lane whose source is outside its row, or whose
// row is masked off, takes the identity.  Every lane must be active.
template <bool MIN>
__device__ __forceinline__ uint32_t wave_scan_dpp(uint32_t x) {
    const int id = MIN ? -1 : 0;
    auto op = [](uint32_t u, int v) { return MIN ? min(u, uint32_t(v)) : u + uint32_t(v); };
    x = op(x, __builtin_amdgcn_update_dpp(id, int(x), 0x111, 0xf, 0xf, false));   // row_shr:1
    x = op(x, __builtin_amdgcn_update_dpp(id, int(x), 0x112, 0xf, 0xf, false));   // row_shr:2
    x = op(x, __builtin_amdgcn_update_dpp(id, int(x), 0x114, 0xf, 0xf, false));   // row_shr:4
    x = op(x, __builtin_amdgcn_update_dpp(id, int(x), 0x118, 0xf, 0xf, false));   // row_shr:8
    x = op(x, __builtin_amdgcn_update_dpp(id, int(x), 0x142, 0xa, 0xf, false));   // row_bcast:15
    x = op(x, __builtin_amdgcn_update_dpp(id, int(x), 0x143, 0xc, 0xf, false));   // row_bcast:31
    return x;
}

// Inclusive prefix sums of x and y over the workgroup; tx / ty receive the
// totals.  lds: 2 * NT / 64 words.
template <uint32_t NT>
__device__ __forceinline__ void block_incl_scan2(uint32_t& x, uint32_t& y, uint32_t* lds, uint32_t& tx,
                                                 uint32_t& ty) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    x = wave_scan_dpp<false>(x);
    y = wave_scan_dpp<false>(y);
    if constexpr (NT == 64) {
        tx = __builtin_amdgcn_readlane(x, 63);
        ty = __builtin_amdgcn_readlane(y, 63);
    } else {
        constexpr int NW = NT / 64;
        if (lane == 63) {
            lds[wave] = x;
            lds[NW + wave] = y;
        }
        __syncthreads();
        uint32_t bx = 0, by = 0;
        #pragma unroll
        for (int w = 0; w < NW; ++w) {
            const uint32_t a = lds[w], b = lds[NW + w];
            bx += w < wave ? a : 0u;
            by += w < wave ? b : 0u;
            tx = w == 0 ? a : tx + a;
            ty = w == 0 ? b : ty + b;
        }
        x += bx;
        y += by;
        __syncthreads();
    }
}

// Workgroup reduction of K values per thread (MIN: minima, else sums);
// every thread receives the results.  lds: NT / 64 * K words.
// Only the values whose bit is set in `active` (uniform) are reduced.
template <uint32_t NT, bool MIN, uint32_t K>
__device__ __forceinline__ void block_reduce(uint32_t (&v)[K], uint32_t* lds, uint64_t active = ~uint64_t(0)) {
    #pragma unroll
    for (uint32_t i = 0; i < K; ++i)
        if ((active >> i) & 1u) v[i] = __builtin_amdgcn_readlane(wave_scan_dpp<MIN>(v[i]), 63);
    if constexpr (NT > 64) {
        constexpr uint32_t NW = NT / 64;
        const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
        if (lane == 0) {
            #pragma unroll
            for (uint32_t i = 0; i < K; ++i)
                if ((active >> i) & 1u) lds[wave * K + i] = v[i];
        }
        __syncthreads();
        #pragma unroll
        for (uint32_t i = 0; i < K; ++i) {
            if (!((active >> i) & 1u)) continue;
            uint32_t s = lds[i];
            #pragma unroll
            for (uint32_t w = 1; w < NW; ++w) s = MIN ? min(s, lds[w * K + i]) : s + lds[w * K + i];
            v[i] = s;
        }
        __syncthreads();
    }
}

// Chunk sizes (pages) a CSR call weighs: thirteen fixed ones and the size
// that gives one wave per wave slot.  An item costs kCsrStartPairs plus its
// page pairs (the planner's cost model for wave items).
constexpr uint32_t kCsrFixedCandidates = 13, kCsrStartPairs = 3, kCsrMaxStates = 64;

__device__ __forceinline__ uint32_t csr_candidate(uint32_t i) {
    switch (i) {
    case 0: return 1u;
    case 1: return 2u;
    case 2: return 4u;
    case 3: return 8u;
    case 4: return 16u;
    case 5: return 32u;
    case 6: return 48u;
    case 7: return 64u;
    case 8: return 96u;
    case 9: return 128u;
    case 10: return 160u;
    case 11: return 192u;
    default: return 256u;
    }
}

__device__ __forceinline__ uint32_t csr_cost(uint32_t pages) { return kCsrStartPairs + (pages + 1) / 2; }

// Common prefix of adjacent sequences (CSR cascade): one wave per (boundary
// b, slice s), b = 1 .. batch - 1, grid-strided.  The boundary's cap is one
// page short of the shorter sequence (each sequence keeps its last page,
// which alone may be partial); slice s covers positions s * kCsrLcpSlice ..
// of it, read 64 ids a load, every load of the slice issued before the
// first compare.  A sequence whose indptr entries are negative or decreasing
// shares nothing.
__global__ __launch_bounds__(256) void csr_lcp_kernel(const int32_t* indptr, const int32_t* indices,
                                                      uint32_t batch, uint32_t page_limit, uint32_t* lcp) {
    constexpr uint32_t U = kCsrLcpSlice / 64;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t nw = gridDim.x * kWaves, total = (batch - 1) * kCsrLcpSlices;
    for (uint32_t w = blockIdx.x * kWaves + (threadIdx.x >> 6); w < total; w += nw) {
        const uint32_t b = 1 + w / kCsrLcpSlices, s = w % kCsrLcpSlices;
        const int32_t a0 = __builtin_amdgcn_readfirstlane(indptr[b - 1]);
        const int32_t a1 = __builtin_amdgcn_readfirstlane(indptr[b]);
        const int32_t b1 = __builtin_amdgcn_readfirstlane(indptr[b + 1]);
        uint32_t cap = 0;
        if (a0 >= 0 && a1 >= a0 && b1 >= a1) {
            const uint32_t m = min(uint32_t(a1 - a0), uint32_t(b1 - a1));
            cap = m ? min(m - 1, DH_MAX_SEQ_LEN / kPageSize - 1) : 0u;
        }
        const uint32_t lo = s * kCsrLcpSlice, hi = min(lo + kCsrLcpSlice, cap);
        uint32_t first = cap, bad = 0xFFFFu;
        if (lo < hi) {
            int32_t x[U], y[U];
            #pragma unroll
            for (uint32_t j = 0; j < U; ++j) {
                const uint32_t pos = lo + 64 * j + lane;
                x[j] = pos < hi ? indices[uint32_t(a0) + pos] : 0;
                y[j] = pos < hi ? indices[uint32_t(a1) + pos] : 0;
            }
            #pragma unroll
            for (int j = int(U) - 1; j >= 0; --j) {   // the lowest sub-block's positions win
                const uint32_t pos = lo + 64 * uint32_t(j) + lane;
                const uint64_t ne = __ballot(pos < hi && x[j] != y[j]);
                const uint64_t bd = __ballot(pos < hi && x[j] == y[j] && uint32_t(x[j]) >= page_limit);
                if (ne) first = lo + 64 * uint32_t(j) + uint32_t(__builtin_ctzll(ne));
                if (bd) bad = lo + 64 * uint32_t(j) + uint32_t(__builtin_ctzll(bd));
            }
            if (bad >= first) bad = 0xFFFFu;
        }
        if (lane == 0) lcp[b * kCsrLcpSlices + s] = first | (bad << 16);
    }
}

// Inclusive max-scan of x over the workgroup in thread order; *tot receives
// the maximum of all.  lds: NT / 64 words.
template <uint32_t NT>
__device__ __forceinline__ uint32_t block_max_scan(uint32_t x, uint32_t* lds, uint32_t& tot) {
    x = ~wave_scan_dpp<true>(~x);
    if constexpr (NT == 64) {
        tot = __builtin_amdgcn_readlane(x, 63);
        return x;
    } else {
        constexpr uint32_t NW = NT / 64;
        const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
        if (lane == 63) lds[wave] = x;
        __syncthreads();
        uint32_t before = 0;
        tot = 0;
        #pragma unroll
        for (uint32_t w = 0; w < NW; ++w) {
            const uint32_t v = lds[w];
            before = w < wave ? max(before, v) : before;
            tot = max(tot, v);
        }
        __syncthreads();
        return max(x, before);
    }
}

// The cascade of a CSR call (LDS): per sequence b (and boundary b, between
// sequences b - 1 and b) and per node.  A node is a run of consecutive
// sequences b0 .. b0 + cnt - 1 and the pages [pd, len) they share: their
// common prefix is at least len pages and their parent node's is pd.  Nodes
// nest as the shared prefixes of a fork tree do (the parent's run holds the
// child's).  Node kinds: group items (kind 1, rows over 64, or over 16 with
// more than 16 pages) or wave items of 16 rows (kind 0, chunks of
// kCsrWaveChunk pages), as the host planner treats shared segments.
constexpr uint32_t kCsrMaxLevels = 4, kCsrMaxNodes = 512, kCsrWaveChunk = 32, kCsrNoDepth = 0xFFFFFFFFu;
struct CsrCascade {
    uint32_t lcp[kCsrCascadeMaxBatch];     // common prefix of b - 1 and b (pages)
    uint32_t bad[kCsrCascadeMaxBatch];     // first shared id outside the pool there (0xFFFF: none)
    uint32_t pd[kCsrCascadeMaxBatch];      // depth of the deepest node holding b - 1 and b (kCsrNoDepth: none)
    uint32_t head[kCsrCascadeMaxBatch];    // run head of b at the current level
    uint32_t tmp[kCsrCascadeMaxBatch];     // scan scratch, later b's first slot
    uint32_t acc[kCsrCascadeMaxBatch];     // at a head: members | 1 << 31 if poisoned
    uint32_t mn[kCsrCascadeMaxBatch];      // at a head: shortest common prefix of its run
    uint32_t skip[kCsrCascadeMaxBatch];    // skip word of b (AttendArgs::csr_skip)
    uint32_t ip[kCsrCascadeMaxBatch];      // indptr[b]
    uint32_t ip_end;                       // indptr[batch]
    uint32_t lv[kCsrMaxLevels][kCsrCascadeMaxBatch];   // node id + 1 of b at a level | slot offset << 16
    uint32_t b0[kCsrMaxNodes], cnt[kCsrMaxNodes], npd[kCsrMaxNodes], len[kCsrMaxNodes];
    uint32_t gc[kCsrMaxNodes], kind[kCsrMaxNodes], item0[kCsrMaxNodes], ss0[kCsrMaxNodes];
    uint32_t nn;
};

// The cascade pass of the CSR planning kernel: nodes level by level from the
// adjacent common prefixes.  At each level a boundary is internal when its
// common prefix reaches kCsrMinShared pages past the depth of the deepest
// node holding both its sequences; maximal runs of internal boundaries are
// the level's nodes, each sharing down to the shortest prefix of its run.
// Group items take chunks of `gchunk` pages: the smallest power of two from
// 8 to 256 whose group items number at most 256 (one per CU), else 256.  A
// node whose shared pages hold a page id outside the pool poisons its
// members (s_bad[b] = 1).  When the items exceed gcap, or the slots leave
// fewer than one per sequence for the rest, nothing is grouped.  Writes the
// skip words (c.skip, p.skip), c.lv and the node records; returns the group
// items, *n_wave the nodes' wave items, *gslots the slots of node chunks.
// The nodes' share of the chip for the chunk choice of the sequences' own
// pages: wave slots they hold, their cost (page pairs plus kCsrStartPairs
// per item, times the waves of an item) and their largest item's cost.
struct CsrNodeLoad {
    uint32_t waves, cost, max_item;
};

template <uint32_t NT>
__device__ uint32_t csr_cascade(const CsrPlanArgs& p, CsrCascade& c, uint32_t* s_bad, uint32_t* red,
                                uint32_t& n_wave, uint32_t& gslots, uint32_t& gchunk, CsrNodeLoad& load) {
    const uint32_t B = p.batch, tid = threadIdx.x;
    // Every slice of a boundary loads at once (one memory round trip), and
    // indptr[b] goes to LDS for the items' page offsets.
    for (uint32_t b = tid; b < B; b += NT) {
        uint32_t mn = 0, bd = 0xFFFFu, v[kCsrLcpSlices];
        c.ip[b] = uint32_t(p.indptr[b]);
        #pragma unroll
        for (uint32_t s = 0; s < kCsrLcpSlices; ++s) v[s] = b > 0 ? p.lcp[b * kCsrLcpSlices + s] : 0u;
        if (b > 0) {
            mn = 0xFFFFu;
            #pragma unroll
            for (uint32_t s = 0; s < kCsrLcpSlices; ++s) {
                mn = min(mn, v[s] & 0xFFFFu);
                bd = min(bd, v[s] >> 16);
            }
        }
        c.lcp[b] = mn;
        c.bad[b] = bd;
        c.pd[b] = b > 0 ? 0u : kCsrNoDepth;
        c.skip[b] = 0u;
        #pragma unroll
        for (uint32_t l = 0; l < kCsrMaxLevels; ++l) c.lv[l][b] = 0u;
    }
    if (tid == 0) {
        c.nn = 0;
        c.ip_end = uint32_t(p.indptr[B]);
    }
    __syncthreads();
    auto internal = [&](uint32_t b) {
        return b > 0 && c.pd[b] != kCsrNoDepth && c.lcp[b] >= c.pd[b] + kCsrMinShared;
    };
    // Each level in one pass over the sequences (in rounds of NT), by
    // scans in thread order: b's run head is the max-scan of the non-internal
    // indices; the run's shortest prefix and first bad id so far are the
    // max-scans of (head << 16 | 0xFFFF - value), whose high half makes the
    // maximum stay inside the run.  A run's last member holds its totals and
    // records the node; its members read the node back from the head.
    uint32_t levels = 0;
    for (uint32_t lev = 0; lev < kCsrMaxLevels; ++lev) {
        for (uint32_t b = tid; b < B; b += NT) c.acc[b] = 0u;
        __syncthreads();
        const uint32_t nn0 = c.nn;
        uint32_t ch = 0, cm = 0, cb = 0, cn = 0;
        for (uint32_t base = 0; base < B; base += NT) {
            const uint32_t b = base + tid;
            const bool valid = b < B, in = valid && internal(b);
            uint32_t th, tm, tb;
            const uint32_t h = max(block_max_scan<NT>(valid && !in ? b : 0u, red, th), ch);
            const uint32_t mv = max(block_max_scan<NT>((h << 16) | (0xFFFFu - (in ? c.lcp[b] : 0xFFFFu)), red, tm), cm);
            const uint32_t bv = max(block_max_scan<NT>((h << 16) | (0xFFFFu - (in ? c.bad[b] : 0xFFFFu)), red, tb), cb);
            const bool last = valid && !(b + 1 < B && internal(b + 1));
            const uint32_t cntb = b - h + 1;
            // A run of fewer than 16 query rows is not worth a node: its
            // sequences read the shared pages themselves (the second read
            // mostly hits the caches), with fewer items and partial states.
            const bool node = last && cntb >= 2u && cntb * p.r >= uint32_t(kWaveRows);
            uint32_t x = node ? 1u : 0u, y = 0, tx, ty;
            block_incl_scan2<NT>(x, y, red, tx, ty);
            const uint32_t k = nn0 + cn + x - 1;
            if (valid) c.head[b] = h;
            if (node && k < kCsrMaxNodes) {
                const uint32_t len = 0xFFFFu - (mv & 0xFFFFu), fb = 0xFFFFu - (bv & 0xFFFFu);
                c.b0[k] = h;
                c.cnt[k] = cntb;
                c.npd[k] = c.pd[h + 1];            // h + 1 is internal: its pd is the run's
                c.len[k] = len;
                c.kind[k] = (lev << 1) | (fb < len ? 1u << 3 : 0u);   // level, poison; kind later
                c.acc[h] = k + 1;
                c.mn[h] = len;
            }
            ch = max(ch, th);
            cm = max(cm, tm);
            cb = max(cb, tb);
            cn += tx;
        }
        __syncthreads();
        if (cn == 0 || nn0 + cn > kCsrMaxNodes) break;   // no node, or too many: stop here
        // Members take the node of their run; boundaries inside a node go one
        // level deeper (their pd becomes the node's shared length).
        for (uint32_t b = tid; b < B; b += NT) {
            const uint32_t h = c.head[b], k1 = c.acc[h];
            c.lv[lev][b] = k1;
            c.tmp[b] = (k1 && internal(b)) ? c.mn[h] : kCsrNoDepth;
        }
        __syncthreads();
        uint32_t deeper[1] = {0u};
        for (uint32_t b = tid; b < B; b += NT) {
            c.pd[b] = c.tmp[b];
            deeper[0] |= (c.tmp[b] != kCsrNoDepth && c.lcp[b] >= c.tmp[b] + kCsrMinShared) ? 1u : 0u;
        }
        block_reduce<NT, false>(deeper, red);
        if (tid == 0) c.nn = nn0 + cn;
        __syncthreads();
        levels = lev + 1;
        if (!deeper[0]) break;   // no boundary reaches a deeper node
    }
    const uint32_t nn = c.nn;
    // Kinds, and the items and slots of each chunk-size candidate.
    constexpr uint32_t NC = 6;
    uint32_t sums[2 * NC + 2] = {};
    const uint32_t GR = p.group_rows;
    for (uint32_t k = tid; k < nn; k += NT) {
        const uint32_t rows = c.cnt[k] * p.r, pages = c.len[k] - c.npd[k];
        const bool grp = rows > 64u || (rows > 16u && pages > 16u);
        c.kind[k] |= grp ? 1u : 0u;
        if (grp) {
            const uint32_t rbk = (rows + GR - 1) / GR;
            #pragma unroll
            for (uint32_t i = 0; i < NC; ++i) {
                const uint32_t g = (pages + (8u << i) - 1) >> (3 + i);
                sums[i] += g * p.hkv * rbk;
                sums[NC + i] += g * c.cnt[k];
            }
        } else {
            const uint32_t g = (pages + kCsrWaveChunk - 1) / kCsrWaveChunk;
            sums[2 * NC] += g * p.hkv * ((rows + kWaveRows - 1) / kWaveRows);
            sums[2 * NC + 1] += g * c.cnt[k];
        }
    }
    block_reduce<NT, false>(sums, red);
    uint32_t pick = NC - 1, items_pick = sums[NC - 1], slots_pick = sums[2 * NC - 1];
    #pragma unroll
    for (int i = int(NC) - 1; i >= 0; --i) {
        if (sums[i] <= 256u) {
            pick = uint32_t(i);
            items_pick = sums[i];
            slots_pick = sums[NC + i];
        }
    }
    const uint64_t need_slots = uint64_t(slots_pick) + sums[2 * NC + 1];
    const bool on = nn > 0 && uint64_t(items_pick) + sums[2 * NC] <= p.gcap && need_slots + B <= p.slot_cap;
    gchunk = on ? 8u << pick : 0u;
    // Per node: chunks, first item (within its kind) and first seqslot; and
    // the load its items put on the chip.
    uint32_t ci = 0, cw = 0, cs = 0;
    uint32_t ld[1] = {0u}, mx[1] = {~0u};
    for (uint32_t base = 0; base < nn; base += NT) {
        const uint32_t k = base + tid;
        uint32_t gi = 0, wi = 0, ss = 0;
        if (on && k < nn) {
            const uint32_t rows = c.cnt[k] * p.r, pages = c.len[k] - c.npd[k];
            const bool grp = c.kind[k] & 1u;
            const uint32_t ch = grp ? gchunk : kCsrWaveChunk;
            const uint32_t g = (pages + ch - 1) / ch, per = p.hkv * (grp ? (rows + GR - 1) / GR
                                                                          : (rows + kWaveRows - 1) / kWaveRows);
            c.gc[k] = g;
            (grp ? gi : wi) = g * per;
            ss = g * c.cnt[k];
            const uint32_t w = grp ? uint32_t(kWaves) : 1u;
            ld[0] += ((g - 1) * csr_cost(ch) + csr_cost(pages - (g - 1) * ch)) * per * w;
            mx[0] = min(mx[0], ~csr_cost(min(ch, pages)));
        }
        uint32_t x = gi, y = wi, tx, ty;
        block_incl_scan2<NT>(x, y, red, tx, ty);
        uint32_t z = ss, zz = 0, tz, tzz;
        block_incl_scan2<NT>(z, zz, red, tz, tzz);
        if (on && k < nn) {
            c.item0[k] = (c.kind[k] & 1u) ? ci + x - gi : cw + y - wi;
            c.ss0[k] = cs + z - ss;
        }
        ci += tx;
        cw += ty;
        cs += tz;
    }
    block_reduce<NT, false>(ld, red);
    block_reduce<NT, true>(mx, red);
    load.waves = on ? ci * kWaves + cw : 0u;
    load.cost = on ? ld[0] : 0u;
    load.max_item = on && mx[0] != ~0u ? ~mx[0] : 0u;
    __syncthreads();
    // Per sequence: shared pages (its deepest node's), node chunks and the
    // slot offset of each level's chunks; poisoned if any node of it is.
    for (uint32_t b = tid; b < B; b += NT) {
        uint32_t depth = 0, chunks = 0;
        bool poison = false;
        for (uint32_t l = 0; l < levels; ++l) {
            const uint32_t k1 = c.lv[l][b] & 0xFFFFu;
            if (!on || !k1) continue;
            const uint32_t k = k1 - 1;
            c.lv[l][b] = k1 | (chunks << 16);
            chunks += c.gc[k];
            depth = c.len[k];
            poison |= (c.kind[k] >> 3) & 1u;
        }
        const uint32_t w = depth ? depth | (chunks << 16) : 0u;
        c.skip[b] = w;
        p.skip[b] = w;
        s_bad[b] = poison ? 1u : 0u;
    }
    __syncthreads();
    n_wave = on ? cw : 0u;
    gslots = on ? cs : 0u;
    if (!on && tid == 0) c.nn = 0;
    __syncthreads();
    return on ? ci : 0u;
}

// Items and seqslot entries of the cascade's nodes (first slots of the
// sequences in c.tmp; seqslot entries from n_chunks on, after the wave
// items' chunks).  Group items of a node cover unit u = chunk * hkv + KV
// head and row block rb; units are taken eight at a time, each with all its
// row blocks eight items apart, so the items reading the same pages run on
// the same XCD (workgroup i runs on XCD i mod 8) and share its L2.  A node's
// wave items (16 rows each) go unit by unit, row blocks within; they follow
// the group items in p.gitems.  red_scratch: the planning kernel's
// reduction space.
template <uint32_t NT>
__device__ void csr_cascade_emit(const CsrPlanArgs& p, const CsrCascade& c, uint32_t n_chunks, uint32_t n_group,
                                 uint32_t gchunk, uint32_t* red_scratch) {
    const uint32_t tid = threadIdx.x, GR = p.group_rows;
    // Seqslots, one thread per sequence: for each node of it (one a level),
    // its slot of every chunk (its first slot, the chunks of its shallower
    // nodes, then the chunk's index) at entry ss0 + chunk * cnt + member.
    for (uint32_t b = tid; b < p.batch; b += NT) {
        #pragma unroll
        for (uint32_t l = 0; l < kCsrMaxLevels; ++l) {
            const uint32_t w = c.lv[l][b], k1 = w & 0xFFFFu;
            if (!k1) continue;
            const uint32_t k = k1 - 1, cnt = c.cnt[k], g = c.gc[k];
            const uint32_t s0 = c.tmp[b] + (w >> 16);
            SeqSlot* dst = p.seqslots + n_chunks + c.ss0[k] + (b - c.b0[k]);
            for (uint32_t chk = 0; chk < g; ++chk) dst[chk * cnt] = SeqSlot{b, s0 + chk};
        }
    }
    // Items: the nodes' items as one range in node order (node k's at
    // s_ws[k] ..), cut into equal contiguous blocks, one a thread.  A thread
    // finds its block's first node by bisection, then walks the nodes'
    // item orders (csr_node_item's) with counters: one division each to
    // start a node, none per item.
    __shared__ uint32_t s_ws[kCsrMaxNodes + 1];
    auto n_items = [&](uint32_t k) {
        const uint32_t rows = c.cnt[k] * p.r;
        return c.gc[k] * p.hkv * ((c.kind[k] & 1u) ? (rows + GR - 1) / GR : (rows + kWaveRows - 1) / kWaveRows);
    };
    uint32_t carry = 0;
    for (uint32_t k0 = 0; k0 < c.nn; k0 += NT) {
        const uint32_t k = k0 + tid;
        const uint32_t v = k < c.nn ? n_items(k) : 0u;
        uint32_t x = v, y = 0u, tx, ty;
        block_incl_scan2<NT>(x, y, red_scratch, tx, ty);
        if (k < c.nn) s_ws[k] = carry + x - v;
        carry += tx;
    }
    if (tid == 0) s_ws[c.nn] = carry;
    __syncthreads();
    const uint32_t total = carry, per = (total + NT - 1) / NT;
    uint32_t f = min(total, tid * per);
    const uint32_t fend = min(total, f + per);
    if (f < fend) {
        uint32_t lo = 0, hi = c.nn;   // the last node starting at or before f
        while (hi - lo > 1) {
            const uint32_t mid = (lo + hi) >> 1;
            if (s_ws[mid] <= f) lo = mid;
            else hi = mid;
        }
        for (uint32_t k = lo; f < fend; ++k) {
            const uint32_t nk0 = s_ws[k], nk1 = s_ws[k + 1];
            if (nk1 <= f) continue;   // an empty node
            const uint32_t b0 = c.b0[k], cnt = c.cnt[k], pd = c.npd[k], len = c.len[k], g = c.gc[k];
            const uint32_t grp = c.kind[k] & 1u, item0 = c.item0[k], ss0 = c.ss0[k], p0 = c.ip[b0];
            const uint32_t rows = cnt * p.r;
            const uint32_t rbk = grp ? (rows + GR - 1) / GR : (rows + kWaveRows - 1) / kWaveRows;
            const uint32_t RR = grp ? GR : uint32_t(kWaveRows), ch = grp ? gchunk : kCsrWaveChunk;
            const uint32_t units = g * p.hkv;
            uint32_t i = f - nk0;
            const uint32_t iend = min(fend, nk1) - nk0;
            // Position of item i: group items take units eight at a time
            // (blk), all row blocks of the eight (rb), then the unit within
            // (uu of m); wave items a unit (blk) and its row blocks.
            uint32_t blk, rb, uu, m;
            if (grp) {
                blk = i / (8 * rbk);
                const uint32_t w = i - blk * 8 * rbk;
                m = min(8u, units - blk * 8);
                rb = w / m;
                uu = w - rb * m;
            } else {
                blk = i / rbk;
                rb = i - blk * rbk;
                uu = 0;
                m = 1;
            }
            const uint32_t u0 = grp ? blk * 8 : blk, u = u0 + uu;
            uint32_t chk0 = u0 / p.hkv, h0 = u0 - chk0 * p.hkv;     // unit blk * 8 (group items)
            uint32_t chk = u / p.hkv, h = u - chk * p.hkv;          // the item's unit
            auto next_unit = [&](uint32_t& ck, uint32_t& hh) {
                if (++hh == p.hkv) {
                    hh = 0;
                    ++ck;
                }
            };
            Item* out = p.gitems + (grp ? 0u : n_group) + item0;
            for (; i < iend; ++i) {
                Item it;
                it.page_off = p0 + pd + chk * ch;
                it.npages = min(ch, len - pd - chk * ch);
                it.seq_off = n_chunks + ss0 + chk * cnt;
                it.row_begin = rb * RR;
                it.nrows = min(RR, rows - rb * RR);
                it.kv_head = h;
                it.flags = 0u;
                it.tail_seq = b0;
                out[i] = it;
                // the next item's position
                if (grp) {
                    next_unit(chk, h);
                    if (++uu == m) {
                        uu = 0;
                        chk = chk0;
                        h = h0;
                        if (++rb == rbk) {
                            rb = 0;
                            for (uint32_t t = 0; t < m; ++t) next_unit(chk0, h0);
                            chk = chk0;
                            h = h0;
                            ++blk;
                            m = min(8u, units - min(units, blk * 8));
                        }
                    }
                } else if (++rb == rbk) {
                    rb = 0;
                    next_unit(chk, h);
                }
            }
            f = min(fend, nk1);
        }
    }
}

// Work decomposition of one dh_decode_csr call, on the device: sequence b's
// pages indptr[b] .. indptr[b+1] split into chunks of `chunk` pages (the last
// one shorter), chunk k of b in partial-state slot slot_ptr[b] + k.
//
// chunk: of the candidates whose chunks fit the workspace's slots, the one
// whose heaviest-first list schedule over kCsrWaveSlots wave slots is
// estimated to end first (ties: the larger chunk, fewer partial states).  The
// estimate is the largest item when the waves fit the slots at once, else
// the mean load plus the smallest item (the last ones placed), at least the
// largest item.  On 35 batches of 1-600 sequences it picks a chunk whose
// exact heaviest-first schedule ends 3 % after the best candidate's on
// average.  Chunks that give a sequence more than kCsrMaxStates partial
// states come last (C2, six 272-page sequences: 4-page chunks, 68 states a
// row, took the merge from the vector to the scalar path).  No candidate
// fitting (more chunks of kCsrMaxChunk pages than the workspace holds):
// overflow, no items, zeros out.
//
// Dispatch order (seqslots[j] = {sequence, slot} of the j-th chunk, j the
// wave item's index / per_chunk): the full chunks first, then the shorter
// last chunks by size, longest first, so the hardware's in-order dispatch
// to free slots is a heaviest-first list schedule.  Order does not change
// results: each chunk's partial state has its slot, merged in slot order.
//
// A sequence whose indptr entries are negative or decreasing, or that has
// more than DH_MAX_SEQ_LEN / 16 pages, gets no chunk and is marked bad
// (zeros out, status DH_EINVAL).
template <uint32_t NT>
__global__ __launch_bounds__(NT) void csr_plan_kernel(CsrPlanArgs p) {
    constexpr uint32_t KC = kCsrFixedCandidates, KM = KC + 1;
    __shared__ uint32_t red[(NT / 64) * 2 * KM];
    __shared__ uint32_t s_tail[kCsrMaxChunk];    // last chunks of each size, then their next position
    // Cascade: its nodes and per-sequence state; members of poisoned nodes.
    __shared__ CsrCascade cc;
    __shared__ uint32_t s_bad[kCsrCascadeMaxBatch];
    const uint32_t tid = threadIdx.x;
    constexpr uint32_t kMaxSeqPages = DH_MAX_SEQ_LEN / kPageSize;
    const uint32_t iters = (p.batch + NT - 1) / NT;
    // Shared prefixes of consecutive sequences first (nodes read by group or
    // multi-sequence wave items): each sequence's own wave items then cover
    // only the pages past its deepest node's.
    const bool casc = p.lcp != nullptr && p.batch >= 2 && p.batch <= kCsrCascadeMaxBatch;
    uint32_t n_gitems = 0, n_nwave = 0, gslots = 0, gchunk = 0;
    CsrNodeLoad nload{0u, 0u, 0u};
    if (casc) n_gitems = csr_cascade<NT>(p, cc, s_bad, red, n_nwave, gslots, gchunk, nload);
    const bool grouped = gslots > 0;
    auto load = [&](uint32_t b, bool& ok) -> uint32_t {
        ok = false;
        if (b >= p.batch) return 0u;
        // With a cascade indptr is in LDS already (no second round trip).
        const int32_t p0 = casc ? int32_t(cc.ip[b]) : p.indptr[b];
        const int32_t p1 = casc ? int32_t(b + 1 < p.batch ? cc.ip[b + 1] : cc.ip_end) : p.indptr[b + 1];
        ok = p0 >= 0 && p1 >= p0 && uint32_t(p1 - p0) <= kMaxSeqPages;
        if (!ok) return 0u;
        return uint32_t(p1 - p0) - (grouped ? (cc.skip[b] & 0xFFFFu) : 0u);
    };
    // Slots the wave items' chunks may take.
    const uint32_t cap_s = p.slot_cap - gslots;
    constexpr uint32_t R = csr_reg_seqs(NT);
    uint32_t nr[R], okr = 0;
    #pragma unroll
    for (uint32_t r = 0; r < R; ++r) {
        bool ok = false;
        nr[r] = load(r * NT + tid, ok);
        okr |= ok ? 1u << r : 0u;
    }
    // f(b, n, ok) over this thread's sequences in order, with a trip count
    // uniform over the workgroup (f may hold barriers); b >= batch: n = 0.
    auto each = [&](auto&& f) {
        #pragma unroll
        for (uint32_t r = 0; r < R; ++r)
            if (r < iters) f(r * NT + tid, nr[r], ((okr >> r) & 1u) != 0u);
        if constexpr (NT > kCsrSmallThreads) {
            for (uint32_t it = R; it < iters; ++it) {
                bool ok = false;
                const uint32_t b = it * NT + tid;
                const uint32_t n = load(b, ok);
                f(b, n, ok);
            }
        }
    };
    for (uint32_t i = tid; i < kCsrMaxChunk; i += NT) s_tail[i] = 0u;

    // Pass 1: pages in all (<= 2^16 * 2^13; the costs below, at most 4 a
    // page, fit 32 bits) and the longest sequence.
    uint32_t tot[1] = {0u}, nmax[1] = {~0u};
    each([&](uint32_t, uint32_t n, bool) {
        tot[0] += n;
        nmax[0] = min(nmax[0], ~n);
    });
    block_reduce<NT, false>(tot, red);
    block_reduce<NT, true>(nmax, red);
    const uint32_t total = tot[0], maxn = ~nmax[0];
    const uint32_t want = uint32_t(min(uint64_t(kCsrMaxChunk),
                                       max(uint64_t(1), (uint64_t(total) * p.per_chunk + kCsrWaveSlots - 1) /
                                                            kCsrWaveSlots)));
    // Candidates weighed (bit i: fixed candidate i; bit KC: want): the fixed
    // sizes from want / 8 up to want (a larger chunk costs more per item and
    // balances no better than want's; below want / 8 an item start costs
    // more than its pages), the smallest fixed size that leaves a sequence
    // at most kCsrMaxStates states, kCsrMaxChunk (the fallback) and want.
    // Sizes below that smallest one are not weighed: they rank after it
    // (more states a row) and need more slots, and it is at most
    // DH_MAX_SEQ_LEN / 16 / kCsrMaxStates = 128 pages, a fixed candidate.
    const uint32_t need = (maxn + kCsrMaxStates - 1) / kCsrMaxStates;
    uint32_t active = (1u << (KC - 1)) | (want >= need ? 1u << KC : 0u);
    bool need_met = false;
    #pragma unroll
    for (uint32_t i = 0; i < KC; ++i) {
        const uint32_t c = csr_candidate(i);
        if (8 * c >= want && c <= want && c >= need) active |= 1u << i;
        if (!need_met && c >= need) {
            active |= 1u << i;
            need_met = true;
        }
    }
    // Pass 2: per candidate, its chunks, their cost and the cheapest chunk.
    uint32_t sums[2 * KM] = {}, mins[KM];
    #pragma unroll
    for (uint32_t i = 0; i < KM; ++i) mins[i] = ~0u;
    each([&](uint32_t, uint32_t n, bool) {
        if (n == 0) return;
        #pragma unroll
        for (uint32_t i = 0; i < KM; ++i) {
            if (!((active >> i) & 1u)) continue;
            const uint32_t c = i < KC ? csr_candidate(i) : want, full = n / c, t = n - full * c;
            sums[i] += full + (t ? 1u : 0u);
            sums[KM + i] += full * csr_cost(c) + (t ? csr_cost(t) : 0u);
            mins[i] = min(mins[i], csr_cost(t ? t : c));
        }
    });
    block_reduce<NT, false>(sums, red, uint64_t(active) | (uint64_t(active) << KM));
    block_reduce<NT, true>(mins, red, active);

    // Chunks that leave a row more than kCsrMaxStates partial states (the
    // merge kernel's vector path) rank after every other fitting one.  The
    // cascade's node items (nload) hold wave slots and add their cost.
    auto end_of = [&](uint32_t c, uint32_t cnt, uint32_t cost, uint32_t mn) -> uint64_t {
        if (cnt > cap_s) return ~uint64_t(0);
        const uint64_t S = kCsrWaveSlots, mx = max(csr_cost(min(c, maxn)), nload.max_item);
        const uint64_t e = uint64_t(cnt) * p.per_chunk + nload.waves <= S
                               ? mx * S
                               : max(mx * S, uint64_t(cost) * p.per_chunk + nload.cost + uint64_t(mn) * S);
        return c < need ? e | (uint64_t(1) << 62) : e;     // more than kCsrMaxStates chunks of maxn pages
    };
    uint32_t chunk = kCsrMaxChunk, n_chunks = sums[KC - 1];
    uint64_t best = ~uint64_t(0);
    #pragma unroll
    for (uint32_t i = 0; i < KM; ++i) {
        if (!((active >> i) & 1u)) continue;
        const uint32_t c = i < KC ? csr_candidate(i) : want;
        const uint64_t e = end_of(c, sums[i], sums[KM + i], mins[i]);
        if (e < best || (e == best && e != ~uint64_t(0) && c > chunk)) {
            best = e;
            chunk = c;
            n_chunks = sums[i];
        }
    }
    const bool overflow = n_chunks > cap_s;

    // Pass 3: last chunks of each size; those of size t take the positions
    // n_chunks - (last chunks of size <= t) onwards, so the longest follow
    // the full chunks and the shortest end the order.
    each([&](uint32_t, uint32_t n, bool) {
        const uint32_t t = n - (n / chunk) * chunk;
        if (t) atomicAdd(&s_tail[t], 1u);
    });
    __syncthreads();
    {
        uint32_t carry = 0;
        for (uint32_t base = 1; base < chunk; base += NT) {
            const uint32_t t = base + tid;
            uint32_t v = t < chunk ? s_tail[t] : 0u, z = 0u, tv, tz;
            block_incl_scan2<NT>(v, z, red, tv, tz);
            if (t < chunk) s_tail[t] = n_chunks - (carry + v);
            carry += tv;
        }
        __syncthreads();
    }

    // Pass 4: each sequence's first slot (prefix sum of the chunk counts)
    // and its chunks' positions: full chunks after the full chunks of the
    // sequences before it, its last chunk from its size's range.
    // With a cascade, a sequence's slots are its group chunks' (one per
    // chunk of its group's shared pages) and then its wave items' chunks.
    uint32_t carry = 0, carry_t = 0, carry_g = 0;
    each([&](uint32_t b, uint32_t n, bool ok) {
        const uint32_t full = n / chunk, t = n - full * chunk, has_t = t ? 1u : 0u, cnt = full + has_t;
        const uint32_t gcb = (grouped && b < p.batch) ? cc.skip[b] >> 16 : 0u;
        uint32_t x = cnt + gcb, y = has_t, tx, ty;
        block_incl_scan2<NT>(x, y, red, tx, ty);
        uint32_t xg = gcb, yg = 0, txg = 0, tyg;
        if (grouped) block_incl_scan2<NT>(xg, yg, red, txg, tyg);
        const uint32_t first = carry + x - cnt - gcb;
        const uint32_t fpos = first - (carry_g + xg - gcb) - (carry_t + y - has_t);
        if (b < p.batch) {
            p.slot_ptr[b] = first;
            p.seq_bad[b] = (ok && !overflow && !(grouped && s_bad[b])) ? 0u : 1u;
            if (grouped) cc.tmp[b] = first;
            if (!overflow && t) {
                const uint32_t pos = atomicAdd(&s_tail[t], 1u);
                if (pos < p.slot_cap) p.seqslots[pos] = SeqSlot{b, first + gcb + full};
            }
        }
        // Full chunks: each lane its own sequence's, or, in the one-wave
        // variant when a sequence has more of them than there are
        // sequences, the whole wave one sequence's after another.
        bool by_wave = false;
        if constexpr (NT == kCsrSmallThreads)
            by_wave = ~uint32_t(__builtin_amdgcn_readlane(wave_scan_dpp<true>(~full), 63)) > p.batch;
        if (!overflow && by_wave) {
            for (uint32_t sq = 0; sq < p.batch; ++sq) {
                const uint32_t fs = __builtin_amdgcn_readlane(full, sq), ps = __builtin_amdgcn_readlane(fpos, sq);
                const uint32_t ss = __builtin_amdgcn_readlane(first + gcb, sq);
                for (uint32_t k = tid; k < fs && ps + k < p.slot_cap; k += kCsrSmallThreads)
                    p.seqslots[ps + k] = SeqSlot{sq, ss + k};
            }
        } else if (!overflow && b < p.batch) {
            for (uint32_t k = 0; k < full && fpos + k < p.slot_cap; ++k)
                p.seqslots[fpos + k] = SeqSlot{b, first + gcb + k};
        }
        carry += tx;
        carry_t += ty;
        carry_g += txg;
    });
    // The nodes' items and seqslots (entries n_chunks .. n_chunks + gslots,
    // after the wave items' chunks in dispatch order).
    const bool emit = grouped && !overflow;
    if (emit) {
        __syncthreads();   // first slots (cc.tmp) of every sequence
        csr_cascade_emit<NT>(p, cc, n_chunks, n_gitems, gchunk, red);
    }
    if (tid == 0) {
        const uint32_t slots = n_chunks + gslots;
        p.slot_ptr[p.batch] = overflow ? 0u : slots;
        p.hdr->chunk = chunk;
        p.hdr->n_items = overflow ? 0u : n_chunks * p.per_chunk;
        p.hdr->overflow = overflow ? 1u : 0u;
        p.hdr->n_chunks = slots;
        p.hdr->n_group = emit ? n_gitems : 0u;
        p.hdr->group_chunk = gchunk;
        p.hdr->n_node_waves = emit ? n_nwave : 0u;
    }
}

// Element-wise two-state merge with natural-log LSE (cascade.rs:116-124).
__global__ __launch_bounds__(256) void merge_states_kernel(const float* o_a, const float* lse_a,
                                                           const float* o_b, const float* lse_b,
                                                           float* o_out, float* lse_out,
                                                           uint32_t n_rows, uint32_t d) {
    const uint64_t idx = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const bool valid = idx < uint64_t(n_rows) * d;
    const uint32_t row = valid ? uint32_t(idx / d) : 0u;
    const uint32_t col = valid ? uint32_t(idx - uint64_t(row) * d) : 1u;
    float res = 0.f, lse = kNegInf;
    if (valid) {
        const float la = lse_a[row], lb = lse_b[row];
        const float mx = fmaxf(la, lb);
        if (mx != kNegInf) {
            const float ea = expf(la - mx), eb = expf(lb - mx);
            const float sum = ea + eb;
            res = (o_a[idx] * ea + o_b[idx] * eb) / sum;
            lse = mx + logf(sum);
        }
    }
    __syncthreads();  // every read of this block's rows precedes the writes (outputs may alias inputs)
    if (valid) {
        o_out[idx] = res;
        if (col == 0) lse_out[row] = lse;
    }
}

// Copies the K and V planes of one KV head for a list of pages.
__global__ __launch_bounds__(256) void gather_kernel(const uint8_t* kv, const uint32_t* pages,
                                                     uint32_t n_pages, uint32_t kv_head, uint32_t hkv,
                                                     uint32_t head_dim, uint32_t eb, uint8_t* out) {
    const uint32_t plane = blockIdx.y;                 // 0 = K, 1 = V
    const uint32_t pi = blockIdx.x;
    const uint64_t bytes = uint64_t(kPageSize) * head_dim * eb;
    const uint8_t* src = kv + plane_offset(pages[pi], plane, kv_head, hkv, head_dim, eb);
    uint8_t* dst = out + (uint64_t(plane) * n_pages + pi) * bytes;
    for (uint64_t i = threadIdx.x * 4; i < bytes; i += blockDim.x * 4)
        *reinterpret_cast<uint32_t*>(dst + i) = *reinterpret_cast<const uint32_t*>(src + i);
}

// The decode kernels' E4M3 -> bf16 conversion, exposed for an exhaustive
// test: codes[4i..4i+3] are scaled by the E8M0 byte e8m0[i].
__global__ __launch_bounds__(256) void e4m3_debug_kernel(const uint32_t* codes, const uint8_t* e8m0,
                                                         uint32_t n4, uint32_t* out) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    uint32_t lo, hi;
    e4m3x4_to_bf16(codes[i], e8m0_to_float(e8m0[i]), lo, hi);
    out[2 * i] = lo;
    out[2 * i + 1] = hi;
}

// Scatters n records of rec bytes from a packed staging buffer to dst[ids[i]].
__global__ __launch_bounds__(256) void scatter_kernel(uint8_t* dst, const uint8_t* src,
                                                      const uint32_t* ids, uint64_t rec) {
    const uint8_t* s = src + uint64_t(blockIdx.x) * rec;
    uint8_t* d = dst + uint64_t(ids[blockIdx.x]) * rec;
    if ((rec & 15) == 0) {
        for (uint64_t o = uint64_t(threadIdx.x) * 16; o < rec; o += uint64_t(blockDim.x) * 16)
            *reinterpret_cast<u32x4*>(d + o) = *reinterpret_cast<const u32x4*>(s + o);
    } else {
        for (uint64_t o = uint64_t(threadIdx.x) * 4; o < rec; o += uint64_t(blockDim.x) * 4)
            *reinterpret_cast<uint32_t*>(d + o) = *reinterpret_cast<const uint32_t*>(s + o);
    }
}

template <int D>
hipError_t launch_prefill_d(const AttendArgs& a, uint32_t n, uint32_t q_dtype, uint32_t kvf, hipStream_t s) {
    dim3 grid(n), block(kWaves * 64);
    if (q_dtype == 1 && kvf == KVF_BF16) {
        hipLaunchKernelGGL((prefill16_kernel<D, KVF_BF16, false>), grid, block, 0, s, a);
    } else if (q_dtype == 0 && kvf == KVF_F16) {
        hipLaunchKernelGGL((prefill16_kernel<D, KVF_F16, true>), grid, block, 0, s, a);
    } else if constexpr (D >= 128) {
        if (q_dtype == 1 && kvf == KVF_FP8) hipLaunchKernelGGL((prefill16_kernel<D, KVF_FP8, false>), grid, block, 0, s, a);
        else if (q_dtype == 1 && kvf == KVF_MX) hipLaunchKernelGGL((prefill16_kernel<D, KVF_MX, false>), grid, block, 0, s, a);
        else if (q_dtype == 0 && kvf == KVF_FP8) hipLaunchKernelGGL((prefill16_kernel<D, KVF_FP8, true>), grid, block, 0, s, a);
        else if (q_dtype == 0 && kvf == KVF_MX) hipLaunchKernelGGL((prefill16_kernel<D, KVF_MX, true>), grid, block, 0, s, a);
        else return hipErrorInvalidValue;
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int D>
hipError_t launch_attend_d(const AttendArgs& a, uint32_t n, uint32_t q_dtype, uint32_t kvf,
                           hipStream_t s) {
    dim3 grid(n), block(kWaves * 64);
    if (q_dtype == 2 && kvf == KVF_F32) {
        hipLaunchKernelGGL(attend32_kernel<D>, grid, block, 0, s, a);
    } else if (q_dtype == 1 && kvf == KVF_BF16) {
        hipLaunchKernelGGL((attend16_kernel<D, KVF_BF16, false>), grid, block, 0, s, a);
    } else if (q_dtype == 1 && kvf == KVF_FP8) {
        hipLaunchKernelGGL((attend16_kernel<D, KVF_FP8, false>), grid, block, 0, s, a);
    } else if (q_dtype == 1 && kvf == KVF_MX) {
        hipLaunchKernelGGL((attend16_kernel<D, KVF_MX, false>), grid, block, 0, s, a);
    } else if (q_dtype == 0 && kvf == KVF_FP8) {   // f16 queries: codes into f16, f16 MFMAs
        hipLaunchKernelGGL((attend16_kernel<D, KVF_FP8, true>), grid, block, 0, s, a);
    } else if (q_dtype == 0 && kvf == KVF_MX) {
        hipLaunchKernelGGL((attend16_kernel<D, KVF_MX, true>), grid, block, 0, s, a);
    } else if (q_dtype == 0 && kvf == KVF_F16) {
        hipLaunchKernelGGL((attend16_kernel<D, KVF_F16, true>), grid, block, 0, s, a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int D>
hipError_t launch_merge_d(const MergeArgs& a, uint32_t q_dtype, hipStream_t s) {
    const uint32_t rows = a.batch * a.hq;
    if (rows == 0) return hipSuccess;
    dim3 grid((rows + 3) / 4), block(256);
    // Rows of 17-32 states: the scalar form, one pass of 32.  Otherwise the
    // vector form with loads per pass for the plan's most states per row, so
    // a row loads no state twice; not known on the host (0, the CSR path):
    // chosen per row from its own count.
    const int states = a.max_states > 64 ? 64 : int(a.max_states);
    auto go = [&](auto out_tag) {
        constexpr uint32_t OUT = decltype(out_tag)::value;
        using MS = MergeShape<D, OUT>;
        const int need = (states + MS::SPI - 1) / MS::SPI;
        if (states == 0) hipLaunchKernelGGL((merge_kernel<D, OUT, -1>), grid, block, 0, s, a);
        else if (states > 16 && states <= 32) hipLaunchKernelGGL((merge_kernel<D, OUT, 0>), grid, block, 0, s, a);
        else if (need <= 1) hipLaunchKernelGGL((merge_kernel<D, OUT, 1>), grid, block, 0, s, a);
        else if (need <= 2 && MS::MAX_NV >= 2) hipLaunchKernelGGL((merge_kernel<D, OUT, (MS::MAX_NV >= 2 ? 2 : 1)>), grid, block, 0, s, a);
        else if (need <= 4 && MS::MAX_NV >= 4) hipLaunchKernelGGL((merge_kernel<D, OUT, (MS::MAX_NV >= 4 ? 4 : 1)>), grid, block, 0, s, a);
        else if (need <= 8 && MS::MAX_NV >= 8) hipLaunchKernelGGL((merge_kernel<D, OUT, (MS::MAX_NV >= 8 ? 8 : 1)>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((merge_kernel<D, OUT, MS::MAX_NV>), grid, block, 0, s, a);
    };
    if (q_dtype == 2) go(std::integral_constant<uint32_t, 2>{});
    else if (q_dtype == 1) go(std::integral_constant<uint32_t, 1>{});
    else go(std::integral_constant<uint32_t, 0>{});
    return hipGetLastError();
}

// Partial-state memory of dh_decode_batch_static: DH_STATIC_WORKSPACE_BYTES
// per GPU, held from the library's load to the end of the process.  Host
// code never uses this name as an address (on the host it is a stand-in,
// not device memory); it asks for the array's device address once per GPU
// (static_scratch_address, from dh_create) and passes that pointer.
static __device__ __align__(256) uint8_t scratch[DH_STATIC_WORKSPACE_BYTES];

}  // namespace

int static_scratch_address(void** out) { return int(hipGetSymbolAddress(out, HIP_SYMBOL(scratch))); }

bool attend_supported(uint32_t q_dtype, uint32_t kvf, uint32_t d) {
    if (d != 64 && d != 128 && d != 256) return false;
    return (q_dtype == 2 && kvf == KVF_F32) || (q_dtype == 1 && kvf == KVF_BF16) ||
           (q_dtype <= 1 && kvf == KVF_FP8) || (q_dtype <= 1 && kvf == KVF_MX) ||
           (q_dtype == 0 && kvf == KVF_F16);
}

int launch_attend(const AttendArgs& a, uint32_t n_items, uint32_t q_dtype, uint32_t kvf,
                  uint32_t d, bool prefill, void* stream) {
    if (n_items == 0) return hipSuccess;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (prefill) {
        switch (d) {
            case 64: return launch_prefill_d<64>(a, n_items, q_dtype, kvf, s);
            case 128: return launch_prefill_d<128>(a, n_items, q_dtype, kvf, s);
            case 256: return launch_prefill_d<256>(a, n_items, q_dtype, kvf, s);
            default: return hipErrorInvalidValue;
        }
    }
    switch (d) {
        case 64: return launch_attend_d<64>(a, n_items, q_dtype, kvf, s);
        case 128: return launch_attend_d<128>(a, n_items, q_dtype, kvf, s);
        case 256: return launch_attend_d<256>(a, n_items, q_dtype, kvf, s);
        default: return hipErrorInvalidValue;
    }
}

int launch_csr_lcp(const int32_t* indptr, const int32_t* indices, uint32_t batch, uint32_t page_limit,
                   uint32_t* lcp, void* stream) {
    if (batch < 2) return hipSuccess;
    const uint64_t waves = uint64_t(batch - 1) * kCsrLcpSlices;
    const uint64_t want = (waves + kWaves - 1) / kWaves;
    const uint32_t blocks = uint32_t(want < 1024 ? want : 1024);
    hipLaunchKernelGGL(csr_lcp_kernel, dim3(blocks), dim3(kWaves * 64), 0, reinterpret_cast<hipStream_t>(stream),
                       indptr, indices, batch, page_limit, lcp);
    return hipGetLastError();
}

int launch_csr_plan(const CsrPlanArgs& p, void* stream) {
    if (p.batch == 0 || p.slot_cap <= p.batch) return hipErrorInvalidValue;
    const auto s = reinterpret_cast<hipStream_t>(stream);
    if (p.batch <= kCsrSmallThreads)
        hipLaunchKernelGGL(csr_plan_kernel<kCsrSmallThreads>, dim3(1), dim3(kCsrSmallThreads), 0, s, p);
    else
        hipLaunchKernelGGL(csr_plan_kernel<kCsrThreads>, dim3(1), dim3(kCsrThreads), 0, s, p);
    return hipGetLastError();
}

int launch_merge(const MergeArgs& a, uint32_t q_dtype, uint32_t d, void* stream) {
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (d) {
        case 64: return launch_merge_d<64>(a, q_dtype, s);
        case 128: return launch_merge_d<128>(a, q_dtype, s);
        case 256: return launch_merge_d<256>(a, q_dtype, s);
        default: return hipErrorInvalidValue;
    }
}

int launch_merge_states(const float* o_a, const float* lse_a, const float* o_b, const float* lse_b,
                        float* o_out, float* lse_out, uint32_t n_rows, uint32_t d, void* stream) {
    const uint64_t n = uint64_t(n_rows) * d;
    if (n == 0) return hipSuccess;
    // One block covers whole rows only, so the in-block barrier orders every
    // read of a row before its writes.
    const uint32_t rows_per_block = d >= 256 ? 1u : 256u / d;
    dim3 block(rows_per_block * d);
    dim3 grid((n_rows + rows_per_block - 1) / rows_per_block);
    hipLaunchKernelGGL(merge_states_kernel, grid, block, 0, reinterpret_cast<hipStream_t>(stream),
                       o_a, lse_a, o_b, lse_b, o_out, lse_out, n_rows, d);
    return hipGetLastError();
}

int launch_e4m3_debug(const uint32_t* codes, const uint8_t* e8m0, uint32_t n4, uint32_t* out,
                      void* stream) {
    if (n4 == 0) return hipSuccess;
    hipLaunchKernelGGL(e4m3_debug_kernel, dim3((n4 + 255) / 256), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), codes, e8m0, n4, out);
    return hipGetLastError();
}

int launch_scatter(uint8_t* dst, const uint8_t* src, const uint32_t* ids, uint32_t n,
                   uint64_t rec_bytes, void* stream) {
    if (n == 0) return hipSuccess;
    if (rec_bytes & 3) return hipErrorInvalidValue;
    hipLaunchKernelGGL(scatter_kernel, dim3(n), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       dst, src, ids, rec_bytes);
    return hipGetLastError();
}

int launch_gather(const uint8_t* kv, const uint32_t* pages, uint32_t n_pages, uint32_t kv_head,
                  uint32_t hkv, uint32_t d, uint32_t eb, uint8_t* out, void* stream) {
    if (n_pages == 0) return hipSuccess;
    dim3 grid(n_pages, 2), block(256);
    hipLaunchKernelGGL(gather_kernel, grid, block, 0, reinterpret_cast<hipStream_t>(stream), kv,
                       pages, n_pages, kv_head, hkv, d, eb, out);
    return hipGetLastError();
}

}  // namespace dh
