// gfx950 (CDNA4) kernels of the paged tree-decode attention path.
//
// attend16 / attend32: one workgroup (four wave64s) per work item.  The item
// names a run of 16-token pages, one KV head and up to 32 (16 for f32) query
// rows; the four waves split the run's pages, each keeps an online softmax
// for its rows, and the waves combine their states through LDS into one
// partial state per row.  ReferenceBackend::decode (crates/dendrite-core/src/
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
// FP8 E4M3 pages are converted to bf16 in registers (exact: E4M3 is a subset
// of bf16); the per-(page, head) fp32 scale multiplies the scores (K) and the
// probabilities (V), which equals dequantising every element.  MXFP8 pages
// are converted with their E8M0 group scale by v_cvt_scalef32_pk_bf16_fp8
// (exact: power-of-two scaling).
#include <hip/hip_runtime.h>
#include <math.h>
#include "dh_device.hpp"

namespace dh {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr uint32_t KVF_F16 = 0, KVF_BF16 = 1, KVF_F32 = 2, KVF_FP8 = 3, KVF_MX = 4;
constexpr float kNegInf = -__builtin_inff();

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

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

__device__ __forceinline__ uint32_t pack2(float a, float b, bool f16) {
    if (f16) {
        f16x2 t = {(_Float16)a, (_Float16)b};
        return __builtin_bit_cast(uint32_t, t);
    }
    bf16x2 t = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, t);
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

// Valid tokens of page index i of an item.
__device__ __forceinline__ int page_tokens(const Item& it, uint32_t i, int last_len) {
    if (i >= it.npages) return 0;
    return ((it.flags & kItemTail) && i + 1 == it.npages) ? last_len : kPageSize;
}

__device__ __forceinline__ int item_last_len(const AttendArgs& a, const Item& it) {
    if (!(it.flags & kItemTail) || a.last_page_len == nullptr) return kPageSize;
    int L = a.last_page_len[it.tail_seq];
    return (L <= 0 || L > kPageSize) ? kPageSize : L;
}

// Cross-wave combine.  Each wave holds, per row of its RT tiles of 16 rows,
// (m, l_partial, O) with O[rt][e][i] = element d = (4g+i)*EPL + e of row
// 16*rt + c.  The waves rescale their O to the workgroup's row maximum and
// store it to their own LDS region; the sum over regions, divided by the
// summed l, is the item's partial state.  (Plain stores: LDS float atomics
// are far slower here.)
template <int D, int RT, int EPL>
struct Combine {
    static constexpr int kStride = D + 4;
    float o[kWaves][RT * 16 * kStride];
    float m[kWaves][RT * 16];
    float l[kWaves][RT * 16];
    float inv[RT * 16];
    uint32_t dst[RT * 16];
};

template <int D, int RT, int EPL, typename Smem>
__device__ __forceinline__ void combine_and_store(const AttendArgs& a, const Item& it, Smem& sm,
                                                  int nrt, float (&m)[RT], float (&l)[RT],
                                                  f4 (&O)[RT][EPL]) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, c = lane & 15;
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        float lt = l[rt] + __shfl_xor(l[rt], 16);
        lt += __shfl_xor(lt, 32);
        if (g == 0) {
            sm.m[wave][rt * 16 + c] = rt < nrt ? m[rt] : kNegInf;
            sm.l[wave][rt * 16 + c] = rt < nrt ? lt : 0.f;
        }
    }
    __syncthreads();
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        if (rt >= nrt) break;
        const int row = rt * 16 + c;
        float M = sm.m[0][row];
        #pragma unroll
        for (int w = 1; w < kWaves; ++w) M = fmaxf(M, sm.m[w][row]);
        if (m[rt] == kNegInf) continue;        // this wave saw no token: region unused
        const float w8 = fast_exp2(m[rt] - M);
        float* orow = sm.o[wave] + row * Smem::kStride;
        #pragma unroll
        for (int i = 0; i < 4; ++i) {
            #pragma unroll
            for (int e = 0; e < EPL; e += 4) {
                f4 v = {O[rt][e][i] * w8, O[rt][e + 1][i] * w8, O[rt][e + 2][i] * w8,
                        O[rt][e + 3][i] * w8};
                *reinterpret_cast<f4*>(orow + (4 * g + i) * EPL + e) = v;
            }
        }
    }
    const int nrows = (int)it.nrows;
    if (tid < nrows) {
        float M = sm.m[0][tid];
        for (int w = 1; w < kWaves; ++w) M = fmaxf(M, sm.m[w][tid]);
        float lt = 0.f;
        if (M != kNegInf) {
            for (int w = 0; w < kWaves; ++w) {
                const float mw = sm.m[w][tid];
                if (mw != kNegInf) lt += sm.l[w][tid] * fast_exp2(mw - M);
            }
        }
        uint32_t seq, slot, qh;
        row_target(a, it, tid, seq, slot, qh);
        const uint32_t dst = slot * a.hq + qh;
        a.ws_lse[dst] = lt > 0.f ? M + log2f(lt) : kNegInf;
        sm.inv[tid] = lt > 0.f ? 1.f / lt : 0.f;
        sm.dst[tid] = dst;
    }
    __syncthreads();
    constexpr int Q4 = D / 4;
    for (int idx = tid; idx < nrows * Q4; idx += kWaves * 64) {
        const int row = idx / Q4, dq = idx - row * Q4;
        f4 acc = {0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            if (sm.m[w][row] == kNegInf) continue;
            acc += *reinterpret_cast<const f4*>(sm.o[w] + row * Smem::kStride + 4 * dq);
        }
        *reinterpret_cast<f4*>(a.ws_o + uint64_t(sm.dst[row]) * D + 4 * dq) = acc * sm.inv[row];
    }
}

// ---------------------------------------------------------------- attend16
// q in bf16 (KV bf16 / FP8 E4M3 / MXFP8) or f16 (KV f16); bf16/f16 MFMA.
//
// Each wave walks its pairs of pages with the loads of the next pair in
// flight behind the current pair's math: K of pair i+1 is requested as soon
// as the score MFMAs of pair i have consumed K, V of pair i+1 as soon as the
// PV MFMAs have consumed V, so no extra registers hold a second buffer.

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
    #pragma unroll
    for (int kb = 0; kb < R::KB; ++kb)
        load_dwords<R::KW>(r.k[kb], kp + (c * D + kb * 32 + 8 * g) * EB);
    if constexpr (KVF == KVF_MX) {
        const uint8_t* s = reinterpret_cast<const uint8_t*>(a.scales) +
                           ((uint64_t(page) * 2 + 0) * a.hkv + head) * uint64_t(kPageSize) * R::G;
        #pragma unroll
        for (int kb = 0; kb < R::G; ++kb) r.ksc[kb] = s[c * R::G + kb];
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

// K rows of a page as MFMA A operands (bf16/f16 dwords).
template <int D, uint32_t KVF>
__device__ __forceinline__ void k_operand(const PageRaw<D, KVF>& r, uint32_t (&op)[D / 32][4]) {
    using R = PageRaw<D, KVF>;
    #pragma unroll
    for (int kb = 0; kb < R::KB; ++kb) {
        if constexpr (!R::FP8) {
            #pragma unroll
            for (int w = 0; w < 4; ++w) op[kb][w] = r.k[kb][w];
        } else {
            const float sc = KVF == KVF_MX ? e8m0_to_float(r.ksc[kb]) : 1.f;
            e4m3x4_to_bf16(r.k[kb][0], sc, op[kb][0], op[kb][1]);
            e4m3x4_to_bf16(r.k[kb][1], sc, op[kb][2], op[kb][3]);
        }
    }
}

// V rows of a page (tokens 4g+j, dims c*EPL..) as bf16/f16 dwords; rows of
// tokens at or beyond nt are zero so that garbage past the valid tokens can
// never reach the accumulator (their probabilities are zero).
template <int D, uint32_t KVF>
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
                e4m3x4_to_bf16(ok ? r.v[j][w] : 0u, sc, op[j][2 * w], op[j][2 * w + 1]);
        }
    }
}

// The page loop of one wave for NRT row tiles (1 or 2), so the MFMA and
// softmax sequences carry no per-tile branches.
template <int D, uint32_t KVF, bool F16, int NRT, int RT>
__device__ __forceinline__ void attend16_pages(const AttendArgs& a, const Item& it, uint32_t pb,
                                               uint32_t pe, int g, int c,
                                               const uint32_t (&qB)[RT][D / 32][4], float (&m)[RT],
                                               float (&l)[RT], f4 (&O)[RT][D / 16]) {
    constexpr int KB = D / 32;
    constexpr int EPL = D / 16;
    constexpr int VOW = EPL / 2;
    constexpr bool BLOCK_SCALE = (KVF == KVF_FP8);
    constexpr float kLazy = 8.f;                  // running-max slack (log2 units)

    const int last_len = item_last_len(a, it);
    const uint32_t* pages = a.pages + it.page_off;
    const uint32_t head = it.kv_head;
    const float* bsc = reinterpret_cast<const float*>(a.scales);

    PageRaw<D, KVF> pr[2];
    float ks[2] = {1.f, 1.f}, vs[2] = {1.f, 1.f};
    {
        uint32_t pg[2];
        #pragma unroll
        for (int p = 0; p < 2; ++p) {
            const uint32_t i = 2 * pb + p;
            pg[p] = pages[i < it.npages ? i : it.npages - 1];
        }
        #pragma unroll
        for (int p = 0; p < 2; ++p) {
            load_page_k<D, KVF>(pr[p], a, pg[p], head, g, c);
            if constexpr (BLOCK_SCALE) ks[p] = bsc[(uint64_t(pg[p]) * 2 + 0) * a.hkv + head];
        }
        #pragma unroll
        for (int p = 0; p < 2; ++p) {
            load_page_v<D, KVF>(pr[p], a, pg[p], head, g, c);
            if constexpr (BLOCK_SCALE) vs[p] = bsc[(uint64_t(pg[p]) * 2 + 1) * a.hkv + head];
        }
    }

    for (uint32_t pi = pb; pi < pe; ++pi) {
        const uint32_t i0 = 2 * pi;
        const int n0 = page_tokens(it, i0, last_len);
        const int n1 = page_tokens(it, i0 + 1, last_len);
        // Next pair's pages.  Past the end the loads repeat the last page:
        // issuing them unconditionally keeps one load order on every path,
        // so the wait before the next pair's scores covers K only.
        uint32_t pgn[2];
        #pragma unroll
        for (int p = 0; p < 2; ++p) {
            const uint32_t i = i0 + 2 + p;
            pgn[p] = pages[i < it.npages ? i : it.npages - 1];
        }

        // Scores of both pages for every row tile.
        uint32_t kop[2][KB][4];
        k_operand<D, KVF>(pr[0], kop[0]);
        k_operand<D, KVF>(pr[1], kop[1]);
        f4 s[NRT][2];
        #pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
            s[rt][0] = f4{0.f, 0.f, 0.f, 0.f};
            s[rt][1] = f4{0.f, 0.f, 0.f, 0.f};
            #pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                s[rt][0] = mma16<F16>(kop[0][kb], qB[rt][kb], s[rt][0]);
                s[rt][1] = mma16<F16>(kop[1][kb], qB[rt][kb], s[rt][1]);
            }
        }
        const float f0 = a.scale_log2 * ks[0], f1 = a.scale_log2 * ks[1];
        const float v0s = vs[0], v1s = vs[1];
        // K of the next pair is in flight behind the softmax and PV math.
        #pragma unroll
        for (int p = 0; p < 2; ++p) {
            load_page_k<D, KVF>(pr[p], a, pgn[p], head, g, c);
            if constexpr (BLOCK_SCALE) ks[p] = bsc[(uint64_t(pgn[p]) * 2 + 0) * a.hkv + head];
        }

        // Online softmax per row tile -> probabilities as B operands.
        uint32_t pB[NRT][4];
        const bool full = (n0 == kPageSize) && (n1 == kPageSize);
        #pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
            float x0[4], x1[4];
            #pragma unroll
            for (int i = 0; i < 4; ++i) {
                x0[i] = s[rt][0][i] * f0;
                x1[i] = s[rt][1][i] * f1;
            }
            if (!full) {
                #pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (4 * g + i >= n0) x0[i] = kNegInf;
                    if (4 * g + i >= n1) x1[i] = kNegInf;
                }
            }
            float mx = fmaxf(fmaxf(fmaxf(x0[0], x0[1]), fmaxf(x0[2], x0[3])),
                             fmaxf(fmaxf(x1[0], x1[1]), fmaxf(x1[2], x1[3])));
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            // Lazy rescaling: the reference max only moves when a score
            // exceeds it by more than kLazy, so exp2 stays <= 2^kLazy and the
            // O/l rescale is skipped on most pairs (O / l is unchanged).
            const bool need = mx > m[rt] + kLazy;
            if (__ballot(need)) {
                const float mnew = need ? mx : m[rt];
                const float alpha = (m[rt] == kNegInf) ? 0.f : fast_exp2(m[rt] - mnew);
                m[rt] = mnew;
                l[rt] *= alpha;
                #pragma unroll
                for (int e = 0; e < EPL; ++e) O[rt][e] *= alpha;
            }
            const float muse = (m[rt] == kNegInf) ? 0.f : m[rt];
            float ps = 0.f;
            #pragma unroll
            for (int i = 0; i < 4; ++i) {
                x0[i] = fast_exp2(x0[i] - muse);
                x1[i] = fast_exp2(x1[i] - muse);
                ps += x0[i] + x1[i];
            }
            l[rt] += ps;
            if constexpr (BLOCK_SCALE) {
                #pragma unroll
                for (int i = 0; i < 4; ++i) {
                    x0[i] *= v0s;
                    x1[i] *= v1s;
                }
            }
            pB[rt][0] = pack2(x0[0], x0[1], F16);
            pB[rt][1] = pack2(x0[2], x0[3], F16);
            pB[rt][2] = pack2(x1[0], x1[1], F16);
            pB[rt][3] = pack2(x1[2], x1[3], F16);
        }

        // O^T += V^T P^T over the pair; the V operand of a d-block is shared
        // by all row tiles.
        uint32_t vop[2][4][VOW];
        v_operand<D, KVF>(pr[0], g, n0, vop[0]);
        v_operand<D, KVF>(pr[1], g, n1, vop[1]);
        #pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int w = e >> 1;
            const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
            uint32_t vA[4];
            vA[0] = __builtin_amdgcn_perm(vop[0][1][w], vop[0][0][w], sel);
            vA[1] = __builtin_amdgcn_perm(vop[0][3][w], vop[0][2][w], sel);
            vA[2] = __builtin_amdgcn_perm(vop[1][1][w], vop[1][0][w], sel);
            vA[3] = __builtin_amdgcn_perm(vop[1][3][w], vop[1][2][w], sel);
            #pragma unroll
            for (int rt = 0; rt < NRT; ++rt) O[rt][e] = mma16<F16>(vA, pB[rt], O[rt][e]);
        }
        // V of the next pair.
        #pragma unroll
        for (int p = 0; p < 2; ++p) {
            load_page_v<D, KVF>(pr[p], a, pgn[p], head, g, c);
            if constexpr (BLOCK_SCALE) vs[p] = bsc[(uint64_t(pgn[p]) * 2 + 1) * a.hkv + head];
        }
    }
}

template <int D, uint32_t KVF, bool F16>
__global__ __launch_bounds__(256, D >= 256 ? 1 : 2) void attend16_kernel(AttendArgs a) {
    constexpr int KB = D / 32;                    // 32-dim k-chunks of a score tile
    constexpr int EPL = D / 16;                   // V elements per lane per token
    constexpr int RT = 2;                         // 16-row tiles per wave

    __shared__ Combine<D, RT, EPL> sm;

    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
    // Wave index as a wave-uniform (scalar) value: page-list reads then go
    // through the scalar cache and never wait on the vector loads in flight.
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const Item it = a.items[blockIdx.x];
    const int nrt = (int)((it.nrows + 15) >> 4);

    // Query rows as B operands: lane (g, c) holds row c, dims kb*32 + 8g .. +8.
    uint32_t qB[RT][KB][4];
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const uint32_t row = rt * 16 + c;
        if (rt < nrt && row < it.nrows) {
            uint32_t seq, slot, qh;
            row_target(a, it, row, seq, slot, qh);
            const uint16_t* qp = reinterpret_cast<const uint16_t*>(a.q) + (uint64_t(seq) * a.hq + qh) * D;
            #pragma unroll
            for (int kb = 0; kb < KB; ++kb) load_dwords<4>(qB[rt][kb], qp + kb * 32 + 8 * g);
        } else {
            #pragma unroll
            for (int kb = 0; kb < KB; ++kb) qB[rt][kb][0] = qB[rt][kb][1] = qB[rt][kb][2] = qB[rt][kb][3] = 0u;
        }
    }

    float m[RT], l[RT];
    f4 O[RT][EPL];
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        m[rt] = kNegInf;
        l[rt] = 0.f;
        #pragma unroll
        for (int e = 0; e < EPL; ++e) O[rt][e] = f4{0.f, 0.f, 0.f, 0.f};
    }

    const uint32_t npairs = (it.npages + 1) >> 1;
    const uint32_t pb = (wave * npairs) / kWaves, pe = ((wave + 1) * npairs) / kWaves;
    if (pb < pe) {
        if (nrt == 2) attend16_pages<D, KVF, F16, 2, RT>(a, it, pb, pe, g, c, qB, m, l, O);
        else attend16_pages<D, KVF, F16, 1, RT>(a, it, pb, pe, g, c, qB, m, l, O);
    }

    combine_and_store<D, RT, EPL>(a, it, sm, nrt, m, l, O);
}

// ---------------------------------------------------------------- attend32
// f32 q and f32 KV: v_mfma_f32_16x16x4_f32, one page per step, 16 rows.
//   S^T: A = K[token c][g*D/4 + kb], B = Q[row c][g*D/4 + kb], kb < D/4.
//   O^T: for token group i: A = V[4g+i][c*EPL + e], B = P[row c][4g+i].
template <int D>
__global__ __launch_bounds__(256) void attend32_kernel(AttendArgs a) {
    constexpr int KQ = D / 4;
    constexpr int EPL = D / 16;
    constexpr int RT = 1;

    __shared__ Combine<D, RT, EPL> sm;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, c = lane & 15;
    const Item it = a.items[blockIdx.x];
    const int nrt = 1;

    float qv[KQ];
    {
        const uint32_t row = c;
        if (row < it.nrows) {
            uint32_t seq, slot, qh;
            row_target(a, it, row, seq, slot, qh);
            const float* qp = reinterpret_cast<const float*>(a.q) + (uint64_t(seq) * a.hq + qh) * D + g * KQ;
            load_dwords<KQ>(reinterpret_cast<uint32_t*>(qv), qp);
        } else {
            #pragma unroll
            for (int k = 0; k < KQ; ++k) qv[k] = 0.f;
        }
    }

    float m[RT] = {kNegInf}, l[RT] = {0.f};
    f4 O[RT][EPL];
    #pragma unroll
    for (int e = 0; e < EPL; ++e) O[0][e] = f4{0.f, 0.f, 0.f, 0.f};

    const int last_len = item_last_len(a, it);
    const uint32_t pb = (wave * it.npages) / kWaves, pe = ((wave + 1) * it.npages) / kWaves;
    const uint32_t* pages = a.pages + it.page_off;
    const uint64_t plane_bytes = uint64_t(kPageSize) * D * 4;

    for (uint32_t pi = pb; pi < pe; ++pi) {
        const int n0 = page_tokens(it, pi, last_len);
        const uint8_t* kp = a.kv + plane_offset(pages[pi], 0, it.kv_head, a.hkv, D, 4);
        const uint8_t* vp = kp + uint64_t(a.hkv) * plane_bytes;
        float kv[KQ];
        load_dwords<KQ>(reinterpret_cast<uint32_t*>(kv), kp + (c * D + g * KQ) * 4);
        float vv[4][EPL];
        #pragma unroll
        for (int i = 0; i < 4; ++i) {
            load_dwords<EPL>(reinterpret_cast<uint32_t*>(vv[i]), vp + ((4 * g + i) * D + c * EPL) * 4);
            if (4 * g + i >= n0) {
                #pragma unroll
                for (int e = 0; e < EPL; ++e) vv[i][e] = 0.f;
            }
        }
        f4 s = {0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int k = 0; k < KQ; ++k) s = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[k], qv[k], s, 0, 0, 0);
        float x[4];
        float mx = kNegInf;
        #pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[i] = (4 * g + i < n0) ? s[i] * a.scale_log2 : kNegInf;
            mx = fmaxf(mx, x[i]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
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
            #pragma unroll
            for (int e = 0; e < EPL; ++e)
                O[0][e] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[i][e], x[i], O[0][e], 0, 0, 0);
        }
    }

    combine_and_store<D, RT, EPL>(a, it, sm, nrt, m, l, O);
}

// ------------------------------------------------------------------ merge
// One wave per (sequence, query head): log-sum-exp over the sequence's
// partial states; no partial state -> zeros (backend.rs:218-222).
template <int D, uint32_t OUT>
__global__ __launch_bounds__(256) void merge_kernel(MergeArgs a) {
    constexpr int PL = D / 64;
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.batch * a.hq) return;
    const uint32_t b = row / a.hq, qh = row - b * a.hq;
    const uint32_t s0 = a.slot_ptr[b], s1 = a.slot_ptr[b + 1];
    float M = kNegInf;
    for (uint32_t s = s0; s < s1; ++s) M = fmaxf(M, a.ws_lse[uint64_t(s) * a.hq + qh]);
    float acc[PL];
    #pragma unroll
    for (int k = 0; k < PL; ++k) acc[k] = 0.f;
    float W = 0.f;
    if (M != kNegInf) {
        for (uint32_t s = s0; s < s1; ++s) {
            const float L = a.ws_lse[uint64_t(s) * a.hq + qh];
            if (L == kNegInf) continue;
            const float w = fast_exp2(L - M);
            W += w;
            const float* o = a.ws_o + (uint64_t(s) * a.hq + qh) * D + lane * PL;
            #pragma unroll
            for (int k = 0; k < PL; ++k) acc[k] += w * o[k];
        }
    }
    const float inv = W > 0.f ? 1.f / W : 0.f;
    const uint64_t ob = (uint64_t(b) * a.hq + qh) * D + lane * PL;
    #pragma unroll
    for (int k = 0; k < PL; ++k) {
        const float v = acc[k] * inv;
        if constexpr (OUT == 2) reinterpret_cast<float*>(a.out)[ob + k] = v;
        else if constexpr (OUT == 1) reinterpret_cast<__bf16*>(a.out)[ob + k] = (__bf16)v;
        else reinterpret_cast<_Float16*>(a.out)[ob + k] = (_Float16)v;
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
    if (q_dtype == 2) hipLaunchKernelGGL((merge_kernel<D, 2>), grid, block, 0, s, a);
    else if (q_dtype == 1) hipLaunchKernelGGL((merge_kernel<D, 1>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((merge_kernel<D, 0>), grid, block, 0, s, a);
    return hipGetLastError();
}

}  // namespace

bool attend_supported(uint32_t q_dtype, uint32_t kvf, uint32_t d) {
    if (d != 64 && d != 128 && d != 256) return false;
    return (q_dtype == 2 && kvf == KVF_F32) || (q_dtype == 1 && kvf == KVF_BF16) ||
           (q_dtype == 1 && kvf == KVF_FP8) || (q_dtype == 1 && kvf == KVF_MX) ||
           (q_dtype == 0 && kvf == KVF_F16);
}

int launch_attend(const AttendArgs& a, uint32_t n_items, uint32_t q_dtype, uint32_t kvf,
                  uint32_t d, void* stream) {
    if (n_items == 0) return hipSuccess;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (d) {
        case 64: return launch_attend_d<64>(a, n_items, q_dtype, kvf, s);
        case 128: return launch_attend_d<128>(a, n_items, q_dtype, kvf, s);
        case 256: return launch_attend_d<256>(a, n_items, q_dtype, kvf, s);
        default: return hipErrorInvalidValue;
    }
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
