// flash_fwd.hip — flash-attention forward for MI355X (gfx950, CDNA4, wave64).
//
// Replaces the reference's device kernels flash_attention_fwd_{v2,opt,h64,h64_bn32,h64_causal} and
// the legacy flash_attention_fwd (src/flash_v2.zig:23, src/flash_opt.zig:17, src/flash_h64.zig:21,
// src/flash_h64_bn32.zig:26, src/flash_h64_causal.zig:20, src/kernels.zig:380). Same math:
// O = softmax(scale * Q K^T, causal mask) V per (batch, head) slice, f16 inputs, f32 accumulation,
// f32 output, online softmax over key tiles with the row max/sum rescale of
// src/flash_h64_bn32.zig:139-211 and the final O / l of src/flash_h64_bn32.zig:246-260. P is rounded
// to f16 for the PV product, and every kernel sums those rounded weights for l, so numerator and
// denominator use the same P. (The reference sums the unrounded f32 weights,
// src/flash_h64_bn32.zig:180-185, which biases O by up to 2^-11 |V| when the dominant weights round
// the same way.)
//
// gfx950 formulation, common to both kernel families
//   * One wave owns 32 queries. It computes the transposed score tile S^T = K * Q^T with
//     v_mfma_f32_32x32x16_f16 (A = K rows from LDS, B = Q^T held in VGPRs for the whole sweep).
//     In the 32x32 accumulator layout lane l holds column (query) l%32 and 16 rows (keys)
//     8*(r/4) + 4*(l/32) + r%4, so the softmax row statistics of a query live in one lane pair
//     (l, l^32): max and sum are in-lane ops plus one v_permlane32_swap.
//   * The exponentiated tile P^T is already in the B-operand layout of the PV product
//     O^T += V^T * P^T (registers 0..7 -> keys 0..15, 8..15 -> keys 16..31), so P never touches LDS.
//   * A workgroup has NQ x NS waves: NQ query groups of 32 rows, each of whose key range is split
//     over NS waves. NS > 1 fills the chip on short sequences; the NS partial (m, l, O) triples are
//     merged through LDS with the same rescale rule, and the LDS epilogue also coalesces the f32
//     stores.
//   * Causal: key sub-tiles entirely above the diagonal are skipped per wave, and key blocks past
//     the workgroup's last query are never staged. Heavy (late) query blocks are dispatched first and
//     workgroups of the same heads are kept on one XCD so their K/V stay in that XCD's L2.
//   * exp is v_exp_f32 on log2-scaled scores (scale * log2(e) folded into one multiply).
// The generic family (flash_fwd_body: any 16-byte aligned layout, 64-bit addressing, and element-wise
// variants for unaligned ones) stages K/V through registers and stores V^T transposed in LDS with
// keys permuted so each A-operand fetch is one ds_read_b128. The pipelined family
// (flash_fwd_pipe_body, the fast path) streams K/V with buffer->LDS DMA into a ring and reads V^T
// with ds_read_b64_tr_b16; it is described where it is defined.
//   * Every kernel also exists with a `_bf16` suffix: bf16 Q/K/V, probabilities rounded to bf16 for
//     the PV product, v_mfma_f32_32x32x16_bf16 (an extension; the reference computes in f16 only).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "notcute_flash.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }

// max / sum of x over the lane pair (l, l^32); both lanes get the identical result.
__device__ __forceinline__ float pair_max(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Element type of Q/K/V and of the probabilities fed to the PV product: f16 (BF = false, the
// reference's type) or bf16. Operands travel as 16-bit payloads in half8 registers either way;
// only the MFMA, the f32 -> 16-bit rounding of P and the row-sum dot product differ.
template <bool BF>
__device__ __forceinline__ floatx16 mfma32(half8 a, half8 b, floatx16 c) {
    if constexpr (BF)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
// Two weights rounded (to nearest even) to the element type, packed as one dword.
template <bool BF>
__device__ __forceinline__ half2v round2(float x, float y) {
    if constexpr (BF) {
        const bf16x2 p = {(__bf16)x, (__bf16)y};
        return __builtin_bit_cast(half2v, p);
    } else {
        const half2v p = {(_Float16)x, (_Float16)y};
        return p;
    }
}
// acc + p.x + p.y, with p in the element type (v_dot2c against 1.0 pairs).
template <bool BF>
__device__ __forceinline__ float sum2(half2v p, float acc) {
    if constexpr (BF) {
        const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, p), ones, acc, false);
    } else {
        const half2v ones = {(_Float16)1.0f, (_Float16)1.0f};
        return __builtin_amdgcn_fdot2(p, ones, acc, false);
    }
}
// A 32-key tile's weight sum (per lane, 16 rounded weights) at or above this moves the running max
// to the tile max. f16: a weight that overflows f16 does, which turns the sum of the rounded
// weights infinite. bf16 has f32's range, so weights are held below 2^20 to keep the f32 row sum
// and O accumulators far from overflow.
template <bool BF>
__device__ __forceinline__ float weight_sum_limit() {
    return BF ? 1048576.0f : __builtin_inff();
}

// Position of key kk (block-relative) inside a staged V^T row: swap bits 2 and 3.
__device__ __forceinline__ int vt_pos(int kk) {
    return (kk & ~12) | ((kk & 4) << 1) | ((kk & 8) >> 1);
}

// 8 consecutive f16 values (16 bytes). VEC: one 16-byte load (caller guarantees alignment).
template <bool VEC>
__device__ __forceinline__ u32x4 load8(const uint16_t *p) {
    if constexpr (VEC) {
        return *reinterpret_cast<const u32x4 *>(p);
    } else {
        u32x4 r;
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = uint32_t(p[2 * i]) | (uint32_t(p[2 * i + 1]) << 16);
        return r;
    }
}

// One 16-byte O store, written through to memory at system scope (sc0 sc1) as a streaming (nt)
// access. A kernel's completion writes back every dirty L2 line it left, on the critical path of
// the launch; a written-through O leaves none. Measured on MI355X against a non-temporal
// write-back store: BH=8 S=1024 d=64 causal 6.06 -> 5.87 us, long sequences unchanged (-0.1 %).
__device__ __forceinline__ void store_o(floatx4 *p, floatx4 v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1 nt" ::"v"(p), "v"(v) : "memory");
}

// Agent-scope (sc1) accesses for the pair exchange between workgroups: coherent across the
// device's XCDs, whose L2 caches are not coherent with one another for ordinary accesses, and
// without the L2 writeback / invalidate that an agent-scope fence costs (buffer_wbl2 / buffer_inv).
// Ordering comes from s_waitcnt: a partial's stores have completed before the counter increment
// that announces them, and the partner's partial is loaded only after the counter showed it.
// Measured on MI355X with partners on the same and on different XCDs: every merged value correct.
__device__ __forceinline__ void store_agent(float *p, floatx4 v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_agent(float *p, float2v v) {
    asm volatile("global_store_dwordx2 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
// Both loads issued, then waited for (asm loads are not tracked by the compiler's waits).
__device__ __forceinline__ void load_agent(const float *p4, const float *p2, floatx4 &v4, float2v &v2) {
    asm volatile("global_load_dwordx4 %0, %2, off sc1\n\tglobal_load_dwordx2 %1, %3, off sc1\n\ts_waitcnt vmcnt(0)"
                 : "=&v"(v4), "=&v"(v2)
                 : "v"(p4), "v"(p2)
                 : "memory");
}

template <bool VEC>
__device__ __forceinline__ void store4(float *p, floatx4 v) {
    if constexpr (VEC) {
        store_o(reinterpret_cast<floatx4 *>(p), v);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = v[i];
    }
}

template <int D, int NQ, int NS>
struct Cfg {
    static constexpr int NW = NQ * NS;           // waves per workgroup
    static constexpr int NT = NW * 64;           // threads per workgroup
    static constexpr int BM = 32 * NQ;           // query rows per workgroup
    static constexpr int BN = 32 * NS;           // keys staged per iteration
    static constexpr int DV = D < 32 ? 32 : D;   // V^T rows in LDS (head 16 padded with zero rows)
    static constexpr int MT = DV / 32;           // 32-row output tiles per wave
    static constexpr int KP = D + 8;             // K row pitch in LDS, halves (16 B pad: no bank clash)
    static constexpr int VP = BN + 8;            // V^T row pitch in LDS, halves
    static constexpr int K_BYTES = BN * KP * 2;
    static constexpr int V_BYTES = DV * VP * 2;
    static constexpr int OP = D + 4;             // merge-buffer row pitch, floats
    static constexpr int O_BYTES = NW * 32 * OP * 4;
    static constexpr int STAGE_BYTES = K_BYTES + V_BYTES;
    static constexpr int ML_OFF = STAGE_BYTES > O_BYTES ? STAGE_BYTES : O_BYTES;
    static constexpr int LDS_BYTES = ML_OFF + NW * 32 * 2 * 4;
    static constexpr int KU = BN * (D / 8);         // 16-byte K chunks per staged block
    static constexpr int VU = (BN / 4) * (D / 8);   // V units of 4 keys x 8 columns
    static constexpr int KREG = (KU + NT - 1) / NT;
    static constexpr int VREG = (VU + NT - 1) / NT;
};

template <int D, int NQ, int NS, bool CAUSAL, bool VEC, bool BF>
__device__ __forceinline__ void flash_fwd_body(const nc_flash_kernel_args &a) {
    using C = Cfg<D, NQ, NS>;
    __shared__ __attribute__((aligned(16))) char smem[C::LDS_BYTES];

    if (a.head_dim != (uint64_t)D || a.seq_len == 0) return;  // as src/flash_h64_bn32.zig:40

    const int S = (int)a.seq_len;
    const uint32_t bh = a.batch_heads;
    const uint32_t nqb = a.num_q_blocks;

    // Workgroup -> (head, query block). Consecutive workgroup ids go round-robin to the 8 XCDs;
    // give each XCD a contiguous range of heads and hand out late (heavier, under a causal mask)
    // query blocks first.
    const uint32_t L = blockIdx.x;
    uint32_t head, qb_rev;
    if ((bh & 7u) == 0) {
        const uint32_t hpx = bh >> 3, x = L & 7u, idx = L >> 3;
        head = x * hpx + idx % hpx;
        qb_rev = idx / hpx;
    } else {
        head = L % bh;
        qb_rev = L / bh;
    }
    const int qb = (int)(nqb - 1u - qb_rev);

    const int tid = threadIdx.x;
    const int w = tid >> 6;
    const int lane = tid & 63;
    const int c = lane & 31;
    const int hh = lane >> 5;
    const int qg = w / NS;
    const int s = w % NS;

    const int q0 = qb * C::BM;        // first query of the workgroup
    const int qw0 = q0 + 32 * qg;     // first query of this wave
    const int qrow = qw0 + c;         // this lane's query
    const int qw_last = min(qw0 + 31, S - 1);

    const uint16_t *qbase = a.q + (size_t)head * a.q_stride;
    const uint16_t *kbase = a.k + (size_t)head * a.k_stride;
    const uint16_t *vbase = a.v + (size_t)head * a.v_stride;
    float *obase = a.o + (size_t)head * a.o_stride;
    const size_t qrs = a.q_row_stride, krs = a.k_row_stride, vrs = a.v_row_stride, ors = a.o_row_stride;

    uint16_t *klds = reinterpret_cast<uint16_t *>(smem);
    uint16_t *vlds = reinterpret_cast<uint16_t *>(smem + C::K_BYTES);

    // Q^T B-operand, resident for the whole key sweep: lane (c, hh) holds Q[qrow][16kk + 8hh .. +7].
    half8 qf[D / 16];
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
        u32x4 t = {0u, 0u, 0u, 0u};
        if (qrow < S) t = load8<VEC>(qbase + (size_t)qrow * qrs + 16 * kk + 8 * hh);
        qf[kk] = __builtin_bit_cast(half8, t);
    }

    if constexpr (D < 32) {  // zero V^T rows D..31 once; staging never writes them
        for (int i = tid; i < (32 - D) * C::VP / 2; i += C::NT)
            reinterpret_cast<uint32_t *>(vlds + D * C::VP)[i] = 0u;
    }

    const int kv_end = CAUSAL ? min(S, q0 + C::BM) : S;
    const int nblk = (kv_end + C::BN - 1) / C::BN;

    u32x4 kreg[C::KREG];
    u32x4 vreg[C::VREG][4];

    auto load_block = [&](int blk) {
        const int kb0 = blk * C::BN;
#pragma unroll
        for (int i = 0; i < C::KREG; ++i) {
            const int u = tid + i * C::NT;
            if (C::KU % C::NT == 0 || u < C::KU) {
                const int key = u / (D / 8), ch = u % (D / 8);
                const int kr = kb0 + key;
                u32x4 t = {0u, 0u, 0u, 0u};
                if (kr < S) t = load8<VEC>(kbase + (size_t)kr * krs + 8 * ch);
                kreg[i] = t;
            }
        }
#pragma unroll
        for (int i = 0; i < C::VREG; ++i) {
            const int u = tid + i * C::NT;
            if (C::VU % C::NT == 0 || u < C::VU) {
                const int kq = u / (D / 8), ch = u % (D / 8);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int kr = kb0 + 4 * kq + j;
                    u32x4 t = {0u, 0u, 0u, 0u};
                    if (kr < S) t = load8<VEC>(vbase + (size_t)kr * vrs + 8 * ch);
                    vreg[i][j] = t;
                }
            }
        }
    };

    auto store_block = [&]() {
#pragma unroll
        for (int i = 0; i < C::KREG; ++i) {
            const int u = tid + i * C::NT;
            if (C::KU % C::NT == 0 || u < C::KU) {
                const int key = u / (D / 8), ch = u % (D / 8);
                *reinterpret_cast<u32x4 *>(klds + key * C::KP + 8 * ch) = kreg[i];
            }
        }
#pragma unroll
        for (int i = 0; i < C::VREG; ++i) {
            const int u = tid + i * C::NT;
            if (C::VU % C::NT == 0 || u < C::VU) {
                const int kq = u / (D / 8), ch = u % (D / 8);
                const int pos = vt_pos(4 * kq);
#pragma unroll
                for (int cp = 0; cp < 4; ++cp) {  // column pair (2cp, 2cp+1) of the 8 staged columns
                    const uint32_t w0 = vreg[i][0][cp], w1 = vreg[i][1][cp];
                    const uint32_t w2 = vreg[i][2][cp], w3 = vreg[i][3][cp];
                    u32x2 even = {(w0 & 0xffffu) | (w1 << 16), (w2 & 0xffffu) | (w3 << 16)};
                    u32x2 odd = {(w0 >> 16) | (w1 & 0xffff0000u), (w2 >> 16) | (w3 & 0xffff0000u)};
                    *reinterpret_cast<u32x2 *>(vlds + (8 * ch + 2 * cp) * C::VP + pos) = even;
                    *reinterpret_cast<u32x2 *>(vlds + (8 * ch + 2 * cp + 1) * C::VP + pos) = odd;
                }
            }
        }
    };

    const float sc = a.scale * kLog2e;
    float m = neg_inf();  // running max of log2-scaled scores (same in both lanes of a pair)
    float l = 0.f;        // this lane's partial row sum
    floatx16 o[C::MT];
#pragma unroll
    for (int mt = 0; mt < C::MT; ++mt) o[mt] = floatx16{};

    if (nblk > 0) load_block(0);
    for (int blk = 0; blk < nblk; ++blk) {
        if (blk > 0) __syncthreads();  // every wave is done reading the previous block
        store_block();
        __syncthreads();
        if (blk + 1 < nblk) load_block(blk + 1);  // in flight while this block is computed

        const int kt0 = blk * C::BN + 32 * s;  // this wave's key sub-tile
        bool run = kt0 < S;
        if (CAUSAL) run = run && kt0 <= qw_last;
        if (!run) continue;

        // S^T = K * Q^T over the head dimension.
        floatx16 acc = floatx16{};
        const uint16_t *krow = klds + (32 * s + c) * C::KP + 8 * hh;
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
            const half8 kf = *reinterpret_cast<const half8 *>(krow + 16 * kk);
            acc = mfma32<BF>(kf, qf[kk], acc);
        }

        float p[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) p[r] = acc[r] * sc;
        const bool need_mask = (kt0 + 32 > S) || (CAUSAL && kt0 + 31 > qw0);
        if (need_mask) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = kt0 + 8 * (r >> 2) + 4 * hh + (r & 3);
                const bool masked = key >= S || (CAUSAL && key > qrow);
                if (masked) p[r] = neg_inf();
            }
        }

        float tmax = p[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) tmax = fmaxf(tmax, p[r]);
        tmax = pair_max(tmax);
        const float m_new = fmaxf(m, tmax);
        const float m_use = (m_new == neg_inf()) ? 0.f : m_new;  // fully masked so far: weights 0
        const float alpha = __builtin_amdgcn_exp2f(m - m_use);
#pragma unroll
        for (int r = 0; r < 16; ++r) p[r] = __builtin_amdgcn_exp2f(p[r] - m_use);

        // P rounded to the element type for the PV product; the row sum adds those rounded weights,
        // so numerator and denominator carry the same rounding.
        half8 pf[2];
        float psum = 0.f;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                const half2v h = round2<BF>(p[8 * ks + j], p[8 * ks + j + 1]);
                pf[ks][j] = h[0];
                pf[ks][j + 1] = h[1];
                psum = sum2<BF>(h, psum);
            }
        l = l * alpha + psum;
        m = m_new;
#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt) o[mt] *= alpha;

        // O^T += V^T * P^T.
#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt) {
            const uint16_t *vrow = vlds + (32 * mt + c) * C::VP + 32 * s + 8 * hh;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const half8 vf = *reinterpret_cast<const half8 *>(vrow + 16 * ks);
                o[mt] = mfma32<BF>(vf, pf[ks], o[mt]);
            }
        }
    }

    // Epilogue: per-wave (m, l, O^T) into LDS, merge the NS key splits, normalise, store O rows.
    __syncthreads();
    float *ob = reinterpret_cast<float *>(smem);
    float *mb = reinterpret_cast<float *>(smem + C::ML_OFF);
    float *lb = mb + C::NW * 32;
    const float lt = pair_sum(l);
    {
        float *dst = ob + (w * 32 + c) * C::OP;
#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = 32 * mt + 8 * i + 4 * hh;
                if (d < D) {
                    floatx4 t = {o[mt][4 * i], o[mt][4 * i + 1], o[mt][4 * i + 2], o[mt][4 * i + 3]};
                    *reinterpret_cast<floatx4 *>(dst + d) = t;
                }
            }
        if (hh == 0) {
            mb[w * 32 + c] = m;
            lb[w * 32 + c] = lt;
        }
    }
    __syncthreads();

    constexpr int DC = D / 4;
    for (int u = tid; u < C::BM * DC; u += C::NT) {
        const int qi = u / DC, ch = u % DC;
        const int row = q0 + qi;
        if (row >= S) continue;
        const int base = (qi / 32) * NS * 32 + (qi % 32);  // wave (qg, 0), query qi%32
        float ms = neg_inf();
#pragma unroll
        for (int j = 0; j < NS; ++j) ms = fmaxf(ms, mb[base + 32 * j]);
        floatx4 accv = {0.f, 0.f, 0.f, 0.f};
        float den = 0.f;
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            const float mj = mb[base + 32 * j];
            const float wgt = (NS == 1) ? 1.f : __builtin_amdgcn_exp2f(mj - ms);
            den += wgt * lb[base + 32 * j];
            const floatx4 oj = *reinterpret_cast<const floatx4 *>(ob + (base + 32 * j) * C::OP + 4 * ch);
            accv += wgt * oj;
        }
        floatx4 res = {accv[0] / den, accv[1] / den, accv[2] / den, accv[3] / den};
        store4<VEC>(obase + (size_t)row * ors + 4 * ch, res);
    }
}


// ---------------------------------------------------------------------------------------------
// Pipelined variant (16-byte aligned rows, slices below 2 GiB): K and V stream through an
// NSTAGE-deep LDS ring by direct buffer->LDS loads (buffer_load_dwordx4 ... lds), so no VGPRs or
// ds_write instructions are spent on staging and NSTAGE-1 blocks are always in flight. The buffer
// descriptors cover exactly each slice's active rows, so key rows past seq_len read as zero
// without a branch. K and V keep their row-major layout in LDS with 16-byte chunks XOR-swizzled
// per row against bank conflicts; the Q K^T A-operand is one ds_read_b128 per 16 head columns, and
// the V^T A-operand of the PV product is assembled by ds_read_b64_tr_b16: inside each 16-lane group
// lane m points at V[r0 + m/4][d0 + 4(m%4)], and lane i receives V[r0..r0+3][d0 + i].
// Shared staging (several query groups): one s_barrier per block (no fence), each wave first
// waiting on its own loads of that block. Private staging (one query group, NQ = 1): each wave
// loads and reads only its own key slice, so the loop has no barrier at all.
// A wave's keys in a block are SUB consecutive 32-key sub-tiles, each taken through S^T, softmax
// and PV before the next. Kernels with key-split waves (NS > 1) stage the workgroup's Q rows in LDS
// once instead of every wave loading its group's rows.
// The softmax keeps a lazy running max: weights are formed against the max as it stands and the
// max only moves when a weight overflows (or, before the first tile, when a row has none).
// ---------------------------------------------------------------------------------------------

#define NC_LDS(T) __attribute__((address_space(3))) T

// LDS layout of a staged K or V block: row r (a key), 16-byte chunk ch (8 head columns) stored at
// slot r*CH + (ch ^ f(r)). f is chosen for the two read patterns on gfx950's 64 x 4-byte banks:
//  - K operand (ds_read_b128): 16 consecutive rows at one chunk must cover all sixteen 16-byte
//    slots of a 256-byte bank window;
//  - V^T operand (ds_read_b64_tr_b16): rows r..r+3 (r % 4 == 0) at four consecutive chunks must
//    too, so for 128-byte rows f(r) and f(r+2) differ in bit 2.
template <int D>
struct Swz {
    static constexpr int CH = D / 8;  // 16-byte chunks per row
    __device__ static __forceinline__ int f(int r) {
        if constexpr (CH == 8) {
            const int x = (r >> 1) & 7;
            return ((x & 1) << 2) | (x >> 1);
        } else if constexpr (CH == 4) {
            return (r >> 2) & 3;
        } else {
            return (r >> 3) & 1;
        }
    }
    __device__ static __forceinline__ int slot(int r, int ch) { return r * CH + (ch ^ f(r)); }
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// s_waitcnt vmcnt(n) with lgkmcnt(0), then a plain workgroup barrier (no memory fence, so loads of
// later blocks stay in flight). The asm memory clobber keeps the compiler from moving LDS accesses
// across it.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xf) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));
    asm volatile("s_barrier" ::: "memory");
}

// s_waitcnt vmcnt(N) only (no barrier): the wave's own staged loads of the block it is about to
// use have landed in LDS, and its earlier LDS reads are complete (lgkmcnt(0)).
template <int N>
__device__ __forceinline__ void wait_vm_only() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xf) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));
    asm volatile("" ::: "memory");
}

// An empty asm statement that consumes the K fragments. It only orders the schedule: the V^T reads
// of a tile are issued after its K reads have landed, so their latency hides behind the softmax
// rather than in front of the S^T products.
template <int N>
__device__ __forceinline__ void lds_reads_done(half8 (&k)[N]) {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
        if constexpr (N % 4 != 0) {
            asm volatile("" ::"v"(k[i]));
        } else {
            asm volatile("" ::"v"(k[i]), "v"(k[i + 1]), "v"(k[i + 2]), "v"(k[i + 3]));
        }
    }
}

template <int N>
struct IC {
    static constexpr int value = N;
};

// x from another lane of the same 16-lane row, selected by the DPP control CTRL (quad_perm,
// row_half_mirror, row_newbcast); every lane of the wave must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Calls f(IC<I>{}) for I = B .. E-1 (compile-time loop index).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (B < E) {
        f(IC<B>{});
        static_for<B + 1, E>(f);
    }
}

// Calls f(IC<A>{}) with A = clamp(x, LO, HI) for a uniform x (a chain of scalar branches).
template <int LO, int HI, typename F>
__device__ __forceinline__ void with_clamped(int x, F &&f) {
    if constexpr (LO >= HI) {
        f(IC<HI>{});
    } else {
        if (x <= LO) {
            f(IC<LO>{});
            return;
        }
        with_clamped<LO + 1, HI>(x, f);
    }
}

// s_waitcnt vmcnt(ahead * LPW) [+ s_barrier] for a uniform ahead in [0, MAXA]: the wave's (or,
// with the barrier, every wave's) loads of the block about to be consumed have landed while the
// loads of the `ahead` blocks issued after it may still be in flight.
template <int LPW, int MAXA>
__device__ __forceinline__ void wait_vm_own(int ahead) {
    with_clamped<0, MAXA>(ahead, [](auto ac) { wait_vm_only<decltype(ac)::value * LPW>(); });
}
template <int LPW, int MAXA>
__device__ __forceinline__ void wait_block(int ahead) {
    with_clamped<0, MAXA>(ahead, [](auto ac) { wait_vm_barrier<decltype(ac)::value * LPW>(); });
}

// Every load that writes registers is issued by the compiler, which places its own waits before
// the first use of each result (no asm-issued load leaves the compiler holding a register whose
// data may not have landed). use_now() is an early use of loop-invariant registers: it puts the
// compiler's wait for them at that point, after the prologue, instead of inside the key loop at
// their first real use, where it would also wait on the K/V prefetch issued just before.
template <int N>
__device__ __forceinline__ void use_now(half8 (&r)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" : "+v"(r[i]));
}

// LDS reads at a lane address plus a compile-time byte offset (folded into the instruction's
// 16-bit offset field when it fits).
template <int OFF>
__device__ __forceinline__ half8 lds_load_b128(uint32_t addr) {
    return *reinterpret_cast<const NC_LDS(half8) *>((uintptr_t)(addr + (uint32_t)OFF));
}
// ds_read_b64_tr_b16 through the gfx950 builtin, so the compiler tracks the result like any load.
// The pointer reaches the builtin as a restrict parameter: the scope metadata this leaves on the
// read tells the compiler's wait placement that it does not alias the buffer->LDS loads in flight,
// so it is not made to wait (vmcnt(0)) for the prefetch of later blocks, exactly as for the K
// reads above. The kernels order every read after the staged block it reads by their own waits.
typedef short short4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 read_tr_b64(const NC_LDS(short4v) *__restrict__ p) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<NC_LDS(short4v) *>(p)));
}
template <int OFF>
__device__ __forceinline__ void ds_read_tr(u32x2 &out, uint32_t addr) {
    out = read_tr_b64(reinterpret_cast<const NC_LDS(short4v) *>((uintptr_t)(addr + (uint32_t)OFF)));
}

template <int D, int NQ, int NS, int NSTAGE, int SUB>
struct PipeCfg {
    static constexpr int NW = NQ * NS;
    static constexpr int NT = NW * 64;
    static constexpr int BM = 32 * NQ;
    static constexpr int WK = 32 * SUB;                 // keys per wave per block
    static constexpr int BN = WK * NS;                  // keys staged per block
    static constexpr int CH = D / 8;
    static constexpr int TILE = BN * D * 2;             // bytes of one K (or V) block
    static constexpr int STAGE = 2 * TILE;
    static constexpr int LOADS = 2 * BN * CH / 64;      // wave-level 16-byte load instructions per block
    static_assert(LOADS % NW == 0, "every wave issues the same number of loads per block");
    static constexpr int LPW = LOADS / NW;
    static_assert(NQ != 1 || LPW % 2 == 0, "private staging: each wave loads as many K as V rows");
    static constexpr int RING = NSTAGE * STAGE;
    static constexpr int OP = D + 4;
    static constexpr int O_BYTES = NW * 32 * OP * 4;
    static constexpr int ML_OFF = RING > O_BYTES ? RING : O_BYTES;
    static constexpr bool QLDS = NS > 1;                                   // Q staged once in LDS
    static constexpr int QLOADS = BM * CH / 64;                            // its wave-instructions
    static_assert(!QLDS || QLOADS <= NW || QLOADS % NW == 0, "the waves share the Q loads evenly");
    static constexpr int Q_OFF = ML_OFF + NW * 32 * 2 * 4;
    static constexpr int LDS_BYTES = Q_OFF + (QLDS ? BM * D * 2 : 0);
    static constexpr int MT = D < 32 ? 1 : D / 32;
};

// What one workgroup of the pipelined body computes: query block nqb-1-qb_rev of slice `head`
// (qb_rev counts from the last, heaviest causal block), and L, its index in the launch, which
// decides whether it is in the end-of-grid balancing tail (nc_flash_kernel_args.balance_tail).
struct PipeSlot {
    uint32_t L, head, qb_rev;
};

// The dispatched kernels' mapping of launch index L to its slot. Workgroups are dealt round-robin
// to the 8 XCDs (L mod 8), so with batch_heads a multiple of 8 each XCD takes whole slices
// (batch_heads/8 of them): every K/V slice is read through one XCD's L2. Within an XCD the query
// blocks go heaviest (causal) first.
__device__ __forceinline__ PipeSlot pipe_slot(uint32_t L, uint32_t bh) {
    if ((bh & 7u) == 0) {
        const uint32_t hpx = bh >> 3, x = L & 7u, idx = L >> 3;
        return PipeSlot{L, x * hpx + idx % hpx, idx / hpx};
    }
    return PipeSlot{L, L % bh, L / bh};
}

// LDS the pipelined body needs (the pair-split kernels add a second Q tile and the exchange words).
template <int D, int NQ, int NS, int NSTAGE, int SUB, bool XS>
constexpr int pipe_lds_bytes() {
    using C = PipeCfg<D, NQ, NS, NSTAGE, SUB>;
    return XS ? C::LDS_BYTES + C::BM * D * 2 + 16 : C::LDS_BYTES;
}

// Per-wave timeline stamps, compiled only into the timeline code object (-DNC_TIMELINE; the product
// kernels carry none) and only into the pipelined kernels that use no scratch memory (the pair-split
// kernels exchange their partials through it). With a.scratch set (bit 0 cleared), each wave writes
// NC_TIMELINE_WORDS u64 at a.scratch + (block * waves + wave) * NC_TIMELINE_WORDS:
//   0-3  core-clock counter (s_memtime) at entry, before and after its key loop, and at its end;
//   4    the same counter after a fixed sleep that follows word 3;
//   5, 6 the chip-wide 100 MHz counter (s_memrealtime) read right after words 3 and 4, which gives
//        the wave's clock at its end and places its counter readings on a common timebase (the read
//        takes ~1 us to return and holds the wave's exit until then, after every other reading);
//   7    HW_ID (low 32 bits) and XCC_ID (high 32 bits);
//   8-11 the wave's key block count, query block, head and key-split index;
//   12   with bit 0 of a.scratch set, the 100 MHz counter at entry (else 0): it gives the wave's
//        average clock over its life, for kernels long enough that the clock moves, and holds
//        the wave for the read's ~1 us at its start.
#define NC_TIMELINE_WORDS 13
#ifdef NC_TIMELINE
#define NC_TL_STAMP(var) const uint64_t var = __builtin_amdgcn_s_memtime();
#define NC_TL_START()                                                                                    \
    NC_TL_STAMP(tl_entry)                                                                                \
    const uint64_t tl_rstart = ((uintptr_t)a.scratch & 1) ? __builtin_amdgcn_s_memrealtime() : 0;
#define NC_TL_END()                                                                                      \
    if constexpr (!XS) {                                                                                 \
        const uint64_t tl_end = __builtin_amdgcn_s_memtime(), tl_r0 = __builtin_amdgcn_s_memrealtime();  \
        __builtin_amdgcn_s_sleep(27);                                                                    \
        const uint64_t tl_end2 = __builtin_amdgcn_s_memtime(), tl_r1 = __builtin_amdgcn_s_memrealtime(); \
        if (lane == 0 && a.scratch != nullptr) {                                                         \
            uint64_t *st = reinterpret_cast<uint64_t *>((uintptr_t)a.scratch & ~(uintptr_t)1) +         \
                           ((size_t)L * C::NW + (uint32_t)w) * NC_TIMELINE_WORDS;                        \
            st[0] = tl_entry; st[1] = tl_loop0; st[2] = tl_loop1; st[3] = tl_end; st[4] = tl_end2;       \
            st[5] = tl_r0; st[6] = tl_r1;                                                                \
            st[7] = __builtin_amdgcn_s_getreg((4) | (0 << 6) | (31 << 11)) |                             \
                    ((uint64_t)__builtin_amdgcn_s_getreg((20) | (0 << 6) | (15 << 11)) << 32);           \
            st[8] = (uint64_t)nblk; st[9] = (uint64_t)qblk; st[10] = head; st[11] = (uint64_t)s;         \
            st[12] = tl_rstart;                                                                          \
        }                                                                                                \
    }
#else
#define NC_TL_STAMP(var)
#define NC_TL_START()
#define NC_TL_END()
#endif

// slot_of(batch_heads) gives the workgroup's PipeSlot (called once the arguments are checked).
template <int D, int NQ, int NS, bool CAUSAL, int NSTAGE, int SUB, bool BF, bool XS = false, typename SlotFn>
__device__ __forceinline__ void flash_fwd_pipe_body(const nc_flash_kernel_args &a, char *smem, SlotFn &&slot_of) {
    using C = PipeCfg<D, NQ, NS, NSTAGE, SUB>;
    using SW = Swz<D>;
    static_assert(NSTAGE >= 1 && NSTAGE <= 8, "ring depth");
    static_assert(!XS || (NQ == 1 && NS == 8 && SUB == 1 && CAUSAL), "pair split: causal private staging");
    // XS: a second Q tile (the B workgroup's second query block) and two words for the pair exchange
    // (pipe_lds_bytes sizes the caller's LDS buffer to match).
    constexpr int XS_Q2 = C::LDS_BYTES;
    constexpr int XS_WORDS = XS_Q2 + C::BM * D * 2;

    if (a.head_dim != (uint64_t)D || a.seq_len == 0) return;
    if (XS && a.scratch == nullptr) return;  // the host always passes the pair-exchange buffer

    const int S = (int)a.seq_len;
    const uint32_t bh = a.batch_heads;
    const uint32_t nqb = a.num_q_blocks;
    // More pairs than the counter region holds would put counters inside the partial slots; the
    // host API refuses such shapes (nc_flash_kernel_scratch_bytes), and a by-name launch of one
    // writes nothing.
    if (XS && (uint64_t)bh * (nqb >> 1) > NC_XS_MAX_PAIRS) return;
    const PipeSlot slot = slot_of(bh);
    const uint32_t L = slot.L, head = slot.head, qb_rev = slot.qb_rev;
    const int qb = (int)(nqb - 1u - qb_rev);

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    NC_TL_START()
    const int c = lane & 31;
    const int hh = lane >> 5;
    const int qg = w / NS;
    const int s = w % NS;

    // Pair split (XS, causal private staging): the query blocks p and q = nqb-1-p of a head
    // (p < nqb/2) hold nqb+1 key tiles (32 keys each) between them, and are shared by two
    // workgroups so that neither takes more than about half the heaviest block's tiles.
    //   A (slot 2p):   block q, key tiles [0, kA), kA = ceil(nqb/2): a partial (m, l, O).
    //   B (slot 2p+1): block q, tiles [kA, q] on waves [0, w1) -> the other partial of block q;
    //                  block p, tiles [0, p] on waves [w1, 8) -> final rows of block p.
    //   solo (odd nqb, last slot): the middle block, all its tiles.
    // A and B exchange their partials of block q through the scratch buffer (see the epilogue).
    // Each wave runs over the key tiles tfirst + sin + g*k of its group (g waves); without the
    // split this is tile s + NS*k of the workgroup's block, as before.
    int xs_role = 2, xs_pair = 0, xs_q = 0, xs_p = 0, xs_w1 = NS;
    int qblk = qb, tfirst = 0, tsin = s, tg = NS, ntile = 0;
    if constexpr (XS) {
        const int nq = (int)nqb, np = nq >> 1, kA = (nq + 1) >> 1;
        const int slot = (int)qb_rev;
        if (slot < 2 * np) {
            xs_role = slot & 1;
            xs_pair = slot >> 1;
            xs_p = xs_pair;
            xs_q = nq - 1 - xs_pair;
            if (xs_role == 0) {
                qblk = xs_q;
                ntile = kA;
            } else {
                const int n1 = xs_q + 1 - kA, n2 = xs_p + 1;
                int best = 1 << 30;  // waves for block q's tail: least tiles on the busiest wave
                for (int w1 = 1; w1 < NS; ++w1) {
                    const int t = max((n1 + w1 - 1) / w1, (n2 + NS - w1 - 1) / (NS - w1));
                    if (t < best) {
                        best = t;
                        xs_w1 = w1;
                    }
                }
                if (s < xs_w1) {
                    qblk = xs_q;
                    tfirst = kA;
                    tg = xs_w1;
                    ntile = n1;
                } else {
                    qblk = xs_p;
                    tsin = s - xs_w1;
                    tg = NS - xs_w1;
                    ntile = n2;
                }
            }
        } else {
            qblk = np;  // the middle block of an odd count
            ntile = np + 1;
        }
    }
    const int q0 = qblk * C::BM;
    const int qw0 = q0 + 32 * qg;
    const int qrow = qw0 + c;
    const int qw_last = min(qw0 + 31, S - 1);

    const uint32_t qrb = (uint32_t)a.q_row_stride * 2, krb = (uint32_t)a.k_row_stride * 2;
    const uint32_t vrb = (uint32_t)a.v_row_stride * 2;
    const uint32_t qspan = (uint32_t)((S - 1) * (uint64_t)a.q_row_stride + D) * 2;
    const uint32_t kspan = (uint32_t)((S - 1) * (uint64_t)a.k_row_stride + D) * 2;
    const uint32_t vspan = (uint32_t)((S - 1) * (uint64_t)a.v_row_stride + D) * 2;
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(a.k + (size_t)head * a.k_stride, kspan);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(a.v + (size_t)head * a.v_stride, vspan);
    float *obase = a.o + (size_t)head * a.o_stride;
    const size_t ors = a.o_row_stride;

    // Q^T B-operand (rows past seq_len read as zero), waited for after the prologue. With NS key-split
    // waves per query group, NS waves need the same 32 rows: the workgroup's BM rows are copied once
    // into an LDS tile (1 KB per wave-instruction, same swizzle as K) and read by every wave after
    // one barrier, instead of each wave fetching its group's rows from L2.
    half8 qf[D / 16];
    if constexpr (XS) {
        // Waves 0-3 stage block q's (or the solo block's) 32 rows, waves 4-7 block p's (B only).
        static_assert(C::QLOADS == 4, "one 32-row Q tile is four wave-instructions");
        const int qb_tile = (w < 4 || xs_role != 1) ? (xs_role == 1 ? xs_q : qblk) : xs_p;
        if (w < 4 || xs_role == 1) {
            const __amdgpu_buffer_rsrc_t qrr = make_rsrc(a.q + (size_t)head * a.q_stride, qspan);
            const int p = (w & 3) * 64 + lane;
            const int r = p / C::CH, sl = p % C::CH;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(qrr, (NC_LDS(void) *)(smem + (w < 4 ? C::Q_OFF : XS_Q2) + (w & 3) * 1024),
                                                     16, (uint32_t)(qb_tile * 32 + r) * qrb + (sl ^ SW::f(r)) * 16, 0, 0, 0);
        }
    } else if constexpr (C::QLDS) {
        const __amdgpu_buffer_rsrc_t qrr = make_rsrc(a.q + (size_t)head * a.q_stride, qspan);
        auto q_load = [&](int t) {  // wave-instruction t of the Q tile
            const int p = t * 64 + lane;
            const int r = p / C::CH, sl = p % C::CH;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(qrr, (NC_LDS(void) *)(smem + C::Q_OFF + t * 1024), 16,
                                                     (uint32_t)(q0 + r) * qrb + (sl ^ SW::f(r)) * 16, 0, 0, 0);
        };
        if constexpr (C::QLOADS <= C::NW) {
            if (w < C::QLOADS) q_load(w);
        } else {
#pragma unroll
            for (int i = 0; i < C::QLOADS / C::NW; ++i) q_load(w + C::NW * i);
        }
    } else {
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk)
            qf[kk] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(
                                                   make_rsrc(a.q + (size_t)head * a.q_stride, qspan),
                                                   (uint32_t)qrow * qrb + (16 * kk + 8 * hh) * 2, 0, 0));
    }

    // One query group per workgroup: every wave consumes only its own key slice of each block,
    // so each wave stages that slice itself and the key loop needs no barrier; a wave
    // runs only over the blocks where its slice has visible keys.
    constexpr bool PRIV = (NQ == 1);
    // Non-causal shared staging: co-resident workgroups of equal work, balanced by wave priority at
    // the end of the grid (the step below). Workgroups before the balancing tail run above it
    // (priority 3), which keeps the arbiter's oldest-first order between them and the tail.
    constexpr bool BALANCE = !PRIV && !CAUSAL;
    const bool balancing = BALANCE && a.balance_tail != 0u && (uint64_t)L + a.balance_tail >= gridDim.x;
    if (BALANCE && a.balance_tail != 0u && !balancing) __builtin_amdgcn_s_setprio(3);
    const int kv_end = CAUSAL ? min(S, q0 + C::BM) : S;
    int nblk = (kv_end + C::BN - 1) / C::BN;
    if constexpr (XS) {
        nblk = tsin < ntile ? (ntile - tsin + tg - 1) / tg : 0;
    } else if constexpr (PRIV) {
        const int last_key = (CAUSAL ? min(S - 1, qw_last) : S - 1) - C::WK * s;
        nblk = last_key < 0 ? 0 : last_key / C::BN + 1;
    }
    // First key of the wave's slice in step blk (private staging): key tile tfirst + tsin + tg*blk.
    auto wave_key0 = [&](int blk) { return 32 * (tfirst + tsin + tg * blk); };

    // Staging: wave-instruction t of a block fills 16-byte slots [64t, 64t+64) of the K tile
    // (t < LOADS/2) or of the V tile; the ring stage is a compile-time constant.
    auto issue = [&](int blk, auto stage_c) {
        constexpr int ST = decltype(stage_c)::value;
        char *sbase = smem + ST * C::STAGE;
#pragma unroll
        for (int n = 0; n < C::LPW; ++n) {
            // Shared staging: wave-instructions are dealt round-robin over the waves. Private
            // staging (one query group): wave s loads exactly the rows of its own key slice.
            const int t = PRIV ? (n < C::LPW / 2 ? s * (C::LPW / 2) + n : C::LOADS / 2 + s * (C::LPW / 2) + n - C::LPW / 2)
                               : w + C::NW * n;
            const bool isv = t >= C::LOADS / 2;
            const int tt = isv ? t - C::LOADS / 2 : t;
            const int p = tt * 64 + lane;
            const int r = p / C::CH, sl = p % C::CH;
            const int ch = sl ^ SW::f(r);
            // private staging: row r of the stage is row r - 32s of the wave's 32-key slice
            const uint32_t key = PRIV ? (uint32_t)(wave_key0(blk) + r - C::WK * s) : (uint32_t)(blk * C::BN + r);
            NC_LDS(void) *dst = (NC_LDS(void) *)(sbase + (isv ? C::TILE : 0) + tt * 1024);
            if (isv)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, dst, 16, key * vrb + ch * 16, 0, 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, dst, 16, key * krb + ch * 16, 0, 0, 0);
        }
    };

    // Lane-dependent LDS byte offsets of the MFMA operand reads within stage 0; stages, sub-tiles
    // and the second 16-key half of a sub-tile add compile-time offsets (the swizzle repeats every
    // 16 rows).
    //  K (A operand of S^T): row WK*s + 32j + c, chunk 2kk + hh.
    const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
    uint32_t kaddr[D / 16];
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) kaddr[kk] = lds0 + SW::slot(C::WK * s + c, 2 * kk + hh) * 16;
    //  V^T (A operand of O^T), per (mt, hf): rows WK*s + 32j + 16ks + 8hf + 4*hv + m/4, columns
    //  32mt + 16cg + 4(m%4) .. +3, with 16-lane group G = 2*hv + cg. Head 16 pads O^T to 32 rows:
    //  its lanes for columns 16..31 re-read columns 0..15 (those output rows are dropped).
    const int G = lane >> 4, m = lane & 15, hv = G >> 1, cg = D < 32 ? 0 : (G & 1);
    uint32_t vaddr[C::MT][2];
#pragma unroll
    for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const int r = C::WK * s + 8 * hf + 4 * hv + (m >> 2);
            const int d = 32 * mt + 16 * cg + 4 * (m & 3);
            vaddr[mt][hf] = lds0 + C::TILE + SW::slot(r, d >> 3) * 16 + ((d >> 2) & 1) * 8;
        }
    constexpr int ROW16 = 16 * C::CH * 16;  // bytes of 16 staged rows

    // Log2-domain scale. A negative scale is applied by negating the resident Q operand (exact),
    // a zero scale by a tiny positive one (every score then rounds to weight exp2(0) = 1, as with
    // a zero scale), so the softmax below can assume sc > 0.
    // Row sum of a tile: the weights exactly as rounded into P, added by v_dot2c against 1.0 pairs,
    // so numerator and denominator carry the same rounding. (Dividing by the sum of the unrounded
    // f32 weights, as the reference does, biases O by up to the rounding's relative error, 2^-11 for
    // f16, times |V| whenever the dominant weights round the same way: 7.8e-3 at |V| = 16.)
    // v_dot2c does not execute while an MFMA of the same SIMD is in flight (measured: 8 v_dot2c per
    // 32x32x16 MFMA take longer than both run one after the other, where FMA, exp and the f16
    // packing hide the MFMAs entirely), but it keeps the fewest registers live.
    float sc = a.scale * kLog2e;
    const bool neg_q = sc < 0.f;  // Q is negated once it has landed
    if (neg_q) sc = -sc;
    if (!(sc > 0.f) && sc == 0.f) sc = 1e-30f;
    float mrow = neg_inf();  // running max of sc * score (log2 domain); -inf: none yet
    float neg_m = 0.f;       // -mrow, 0 while mrow is -inf
    float l = 0.f;
    floatx16 o[C::MT];
#pragma unroll
    for (int mt = 0; mt < C::MT; ++mt) o[mt] = floatx16{};

    // K prefetch (private staging, two stages, one sub-tile per step): a wave's next tile is in the
    // other ring stage, and its slice has landed by the end of the current step, so the next K
    // operand is read from LDS right after this tile's PV products are issued and arrives while
    // they run instead of at the head of the next step.
    constexpr bool KPF = PRIV && NSTAGE == 2 && SUB == 1;
    half8 kpf[D / 16];

    // One 32x32 sub-tile of this wave: S^T = K Q^T for its 32 keys (kt0 ..), online softmax, and
    // O^T += V^T P^T. TOFF is the sub-tile's byte offset in the LDS ring (a compile-time constant);
    // with K prefetch, NEXT is the next tile's offset and has_next says whether the wave has one.
    auto tile = [&](const int kt0, auto toff_c, auto next_c, const bool has_next) {
        constexpr int TOFF = decltype(toff_c)::value;
        constexpr int NEXT = decltype(next_c)::value;

        // S^T of the sub-tile.
        floatx16 acc = floatx16{};
        half8 kf[D / 16];
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
            if constexpr (KPF)
                kf[kk] = kpf[kk];
            else
                kf[kk] = lds_load_b128<TOFF>(kaddr[kk]);
            acc = mfma32<BF>(kf[kk], qf[kk], acc);
        }
        lds_reads_done(kf);
        // V^T operands: their latency hides behind the softmax.
        u32x2 vt[C::MT * 4];
#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt) {
            u32x2 *v4 = vt + mt * 4;
            ds_read_tr<TOFF>(v4[0], vaddr[mt][0]);
            ds_read_tr<TOFF>(v4[1], vaddr[mt][1]);
            ds_read_tr<TOFF + ROW16>(v4[2], vaddr[mt][0]);
            ds_read_tr<TOFF + ROW16>(v4[3], vaddr[mt][1]);
        }

        // Online softmax (sc > 0). P = exp2(sc * s - m) is formed against the running max m as it
        // stands and rounded to f16 for the PV product; the row sum adds the rounded weights.
        // f16 keeps its relative precision up to 65504, so m only has to
        // move when some weight overflows f16, which shows in that lane's tile sum (see
        // weight_sum_limit); then (and while a row has no max yet)
        // the tile max is taken - before scaling, exact since rounding is monotonic - O and l
        // are rescaled and the tile is redone. Once a row has a max its sum is >= 1, so small
        // weights cannot underflow it.
        const bool need_mask = (kt0 + 32 > S) || (CAUSAL && kt0 + 31 > qw0);
        if (need_mask) {
            // lim: the last visible key offset in the sub-tile. The shared-staging kernels fold this
            // lane's 4*hh into it, so every element compares against an inline constant and no
            // per-element key offsets stay live across their register-tight key loop; the
            // private-staging kernels have registers to spare and keep the offsets precomputed.
            if constexpr (PRIV) {
                const int lim = CAUSAL ? min(qrow, S - 1) - kt0 : S - 1 - kt0;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (8 * (r >> 2) + 4 * hh + (r & 3) > lim) acc[r] = neg_inf();
            } else {
                const int lim = (CAUSAL ? min(qrow, S - 1) - kt0 : S - 1 - kt0) - 4 * hh;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (8 * (r >> 2) + (r & 3) > lim) acc[r] = neg_inf();
            }
        }
        half8 pf[2];
        auto weights = [&]() {
            {
                float ls = 0.f;
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    half2v h[4];
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        h[t] = round2<BF>(__builtin_amdgcn_exp2f(__builtin_fmaf(acc[8 * ks + 2 * t], sc, neg_m)),
                                          __builtin_amdgcn_exp2f(__builtin_fmaf(acc[8 * ks + 2 * t + 1], sc, neg_m)));
                        pf[ks][2 * t] = h[t][0];
                        pf[ks][2 * t + 1] = h[t][1];
                    }
#pragma unroll
                    for (int t = 0; t < 4; ++t) ls = sum2<BF>(h[t], ls);
                }
                return ls;
            }
        };
        // Move the running max to the tile max (rows whose max does not grow keep it) and rescale.
        auto to_tile_max = [&]() {
            const floatx16 &x = acc;
            const float m0 = fmaxf(fmaxf(x[0], x[1]), x[2]), m1 = fmaxf(fmaxf(x[3], x[4]), x[5]);
            const float m2 = fmaxf(fmaxf(x[6], x[7]), x[8]), m3 = fmaxf(fmaxf(x[9], x[10]), x[11]);
            const float m4 = fmaxf(fmaxf(x[12], x[13]), x[14]);
            // (folding -inf in first lets the compiler fuse the tree into v_max3 without extra
            // canonicalising maxes)
            const float tmax = fmaxf(neg_inf(), fmaxf(fmaxf(fmaxf(m0, m1), m2), fmaxf(fmaxf(m3, m4), x[15])));
            const float m_new = fmaxf(mrow, pair_max(tmax) * sc);
            const float alpha = __builtin_amdgcn_exp2f(mrow - (m_new == neg_inf() ? 0.f : m_new));
            l *= alpha;
#pragma unroll
            for (int mt = 0; mt < C::MT; ++mt) o[mt] *= alpha;
            mrow = m_new;
            neg_m = (mrow == neg_inf()) ? 0.f : -mrow;
        };
        float ls;
        if (__builtin_amdgcn_ballot_w64(mrow == neg_inf())) {
            to_tile_max();  // some row has no max yet: take it first
            ls = weights();
        } else {
            ls = weights();
            if (__builtin_amdgcn_ballot_w64(!(ls < weight_sum_limit<BF>()))) {
                to_tile_max();  // a weight overflowed (f16) or grew too large (bf16): redo the tile
                ls = weights();
            }
        }
        l += ls;

#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const u32x2 *v4 = vt + mt * 4 + 2 * ks;
                const u32x4 vv = {v4[0][0], v4[0][1], v4[1][0], v4[1][1]};
                o[mt] = mfma32<BF>(__builtin_bit_cast(half8, vv), pf[ks], o[mt]);
            }
        if constexpr (KPF) {
            if (has_next) {
                wait_vm_only<0>();  // the wave's slice of the next block has landed
#pragma unroll
                for (int kk = 0; kk < D / 16; ++kk) kpf[kk] = lds_load_b128<NEXT>(kaddr[kk]);
            }
        }
    };
    // One key block: wait for its stage, refill the stage consumed last step, compute this wave's
    // sub-tiles.
    auto step = [&](int blk, auto stage_c) {
        constexpr int ST = decltype(stage_c)::value;
        if constexpr (BALANCE) {
            // The grid's last workgroups (balance_tail of them) share their CUs with each other to
            // the end. The issue arbiter favours older waves, so of two co-resident workgroups with
            // equal work the older finished first and the younger ran its last third alone at half
            // the CU's waves; ordering waves by remaining key blocks (priority 2 above half, 1 above
            // 3/16, else 0) keeps such workgroups level, so they finish together.
            if (balancing) {
                const int rem32 = (nblk - blk) * 32;
                if (rem32 >= 16 * nblk)
                    __builtin_amdgcn_s_setprio(2);
                else if (rem32 >= 6 * nblk)
                    __builtin_amdgcn_s_setprio(1);
                else
                    __builtin_amdgcn_s_setprio(0);
            }
        }
        if constexpr (PRIV && NSTAGE == 1) {
            // Private single stage: the wave's reads of the previous block are complete (their
            // results were consumed), so it refills the stage with this block and waits for it.
            if (blk > 0) issue(blk, IC<0>{});
            wait_vm_only<0>();
        } else if constexpr (KPF) {
            // this block's slice was waited for before its K was prefetched
            if (blk + 1 < nblk) issue(blk + 1, IC<(ST + 1) % 2>{});
        } else if constexpr (PRIV) {
            wait_vm_own<C::LPW, NSTAGE - 2>(min(NSTAGE - 2, nblk - 1 - blk));
            if (blk + NSTAGE - 1 < nblk) issue(blk + NSTAGE - 1, IC<(ST + NSTAGE - 1) % NSTAGE>{});
        } else if constexpr (NSTAGE == 1) {
            // Single stage: refill it once every wave is done with the previous block.
            if (blk > 0) {
                __builtin_amdgcn_s_waitcnt(0xc07f & ~(0xf << 8));  // lgkmcnt(0)
                asm volatile("s_barrier" ::: "memory");
                issue(blk, IC<0>{});
            }
            wait_vm_barrier<0>();
        } else {
            wait_block<C::LPW, NSTAGE - 2>(min(NSTAGE - 2, nblk - 1 - blk));
            if (blk + NSTAGE - 1 < nblk) issue(blk + NSTAGE - 1, IC<(ST + NSTAGE - 1) % NSTAGE>{});
        }

        // The wave's keys in the block are SUB consecutive 32-key sub-tiles, each taken through S^T,
        // softmax and PV before the next (one sub-tile's operands live at a time), so a block of
        // 32*NS*SUB keys costs one wait and one barrier.
        const int kb = PRIV ? wave_key0(blk) : blk * C::BN + C::WK * s;  // the wave's first key in the block
        bool run = kb < S;
        if (CAUSAL) run = run && kb <= qw_last;
        if (!run) return;
        static_for<0, SUB>([&](auto jc) {
            constexpr int TOFF = ST * C::STAGE + 2 * decltype(jc)::value * ROW16;  // sub-tile in the stage
            tile(kb + 32 * decltype(jc)::value, IC<TOFF>{}, IC<((ST + 1) % NSTAGE) * C::STAGE>{}, blk + 1 < nblk);
            __builtin_amdgcn_sched_barrier(0);  // keep sub-tiles (and steps) apart
        });
    };

    // Prologue: blocks 0 .. NSTAGE-2 in flight; then Q (issued before them) has landed once at most
    // their loads are outstanding. With Q in registers (shared staging, where every wave has at
    // least one block) the prologue's blocks are issued whatever nblk is (a block past the keys
    // reads zeros and is never consumed), so the wait count is a constant and the compiler sees Q
    // complete at it.
    static_for<0, (NSTAGE > 1 ? NSTAGE - 1 : 1)>([&](auto ic) {
        constexpr int I = decltype(ic)::value;
        if (!C::QLDS || I < nblk) issue(I, IC<I>{});
    });
    if constexpr (C::QLDS)
        with_clamped<0, (NSTAGE > 1 ? NSTAGE - 1 : 1)>(nblk, [&](auto ac) { wait_vm_only<decltype(ac)::value * C::LPW>(); });
    else
        wait_vm_only<(NSTAGE > 1 ? NSTAGE - 1 : 1) * C::LPW>();
    if constexpr (C::QLDS) {
        asm volatile("s_barrier" ::: "memory");  // every wave's part of the Q tile has landed
        const uint32_t qt = lds0 + ((XS && xs_role == 1 && s >= xs_w1) ? XS_Q2 : C::Q_OFF);
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk)
            qf[kk] = *reinterpret_cast<const NC_LDS(half8) *>((uintptr_t)(qt + SW::slot(32 * qg + c, 2 * kk + hh) * 16));
    }
    use_now(qf);
    if constexpr (KPF) {
        if (nblk > 0) {
            wait_vm_only<0>();  // block 0's slice
#pragma unroll
            for (int kk = 0; kk < D / 16; ++kk) kpf[kk] = lds_load_b128<0>(kaddr[kk]);
        }
    }
    if (neg_q) {
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) qf[kk] = -qf[kk];
    }
    NC_TL_STAMP(tl_loop0)
    for (int blk0 = 0; blk0 < nblk; blk0 += NSTAGE) {
        step(blk0, IC<0>{});
        static_for<1, NSTAGE>([&](auto ic) {
            constexpr int I = decltype(ic)::value;
            if (blk0 + I < nblk) step(blk0 + I, IC<I>{});
        });
    }

    NC_TL_STAMP(tl_loop1)
    constexpr int DC = D / 4;
    float2v *mlb = reinterpret_cast<float2v *>(smem + C::ML_OFF);  // [BM queries][NS splits]
    const float lt = pair_sum(l);
    if constexpr (PRIV && NS > 1) {
        // Epilogue, private staging: once a wave is past its loop, the K and V slices of ring
        // stage 0 that only it ever loaded are free, so it writes its unscaled O^T partial there
        // (queries 0-15 over its K slice, 16-31 over its V slice, 16-byte chunks XOR-swizzled by
        // row) and its (m, l) in the dedicated area, all before the single barrier. Then each output
        // float4 is sum_j w_j o_j / L with w_j = exp2(m_j - M), M = max_j m_j, L = sum_j w_j l_j
        // over the NS key splits (w_j = 0 for a split that saw no key), stored row-contiguously.
        static_assert(SUB == 1, "a wave's staged slice is 32 rows");
        constexpr int SLICE = 64 * D;  // bytes of one wave's 32 staged rows of K (or V)
        auto part = [&](int split, int q, int chunk) {
            const int lr = q & 15;
            return reinterpret_cast<floatx4 *>(smem + (q < 16 ? 0 : C::TILE) + split * SLICE + lr * 4 * D +
                                               ((chunk ^ (lr & (DC - 1))) << 4));
        };
        if (hh == 0) mlb[c * NS + s] = float2v{mrow, lt};
#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = 32 * mt + 8 * i + 4 * hh;
                if (d < D) *part(s, c, d >> 2) = floatx4{o[mt][4 * i], o[mt][4 * i + 1], o[mt][4 * i + 2], o[mt][4 * i + 3]};
            }
        if constexpr (XS) {
            // Pair exchange. Scratch: one u32 counter per pair in a fixed NC_XS_COUNTER_BYTES region,
            // then per pair two slots (A's, B's): 32 x D f32 unnormalised O, then 32 (m, l) pairs.
            // Each workgroup of a pair adds 1 to the counter once per launch, so it is even when a
            // launch starts and odd once one of the two has published its partial. The workgroup
            // that finds it odd merges both partials into O; the other only publishes. Nothing
            // waits on the other workgroup, and the counter needs no reset.
            // Before its barrier, one thread reads the counter: if the partner has already
            // published, this workgroup merges at once (one round trip for the partner's partial)
            // and adds its 1 without waiting for the result. Otherwise it publishes its partial,
            // waits for the stores, adds 1 and merges if the result shows the partner got there in
            // between.
            static_assert(C::NT == 512 && DC == 16 && C::BM == 32, "one thread per (row, 4 columns) of a block");
            constexpr int SLOT = 32 * D * 4 + 32 * 8;
            uint32_t *xw = reinterpret_cast<uint32_t *>(smem + XS_WORDS);
            const uint32_t np = nqb >> 1;
            const size_t pg = (size_t)head * np + (uint32_t)xs_pair;
            uint32_t *cnt = reinterpret_cast<uint32_t *>(a.scratch) + pg;
            char *slots = reinterpret_cast<char *>(a.scratch) + NC_XS_COUNTER_BYTES;
            if (xs_role < 2 && tid == 0) xw[0] = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            wait_vm_barrier<0>();
            const int qi = tid >> 4, ch = tid & 15;
            // (M, L, O) of row qi, columns 4ch..4ch+3, merged over the waves of group 1 (waves
            // [0, w1): block q, or the whole workgroup) and of group 2 (B's waves [w1, 8): block p).
            // Every wave's partial is read once, unconditionally, and split between the groups by
            // selects (branches here serialised the LDS reads).
            const int w1 = xs_role == 1 ? xs_w1 : NS;
            float2v ml[NS];
            floatx4 pj[NS];
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                ml[j] = mlb[qi * NS + j];
                pj[j] = *part(j, qi, ch);
            }
            float M1 = neg_inf(), M2 = neg_inf();
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                if (j < w1)
                    M1 = fmaxf(M1, ml[j][0]);
                else
                    M2 = fmaxf(M2, ml[j][0]);
            }
            float L1 = 0.f, L2 = 0.f;
            floatx4 o1 = {0.f, 0.f, 0.f, 0.f}, o2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                const bool g1 = j < w1;
                const float wj = __builtin_amdgcn_exp2f(ml[j][0] - (g1 ? M1 : M2));  // 0 for a wave without keys
                const float a1 = g1 ? wj : 0.f, a2 = g1 ? 0.f : wj;
                L1 = __builtin_fmaf(a1, ml[j][1], L1);
                L2 = __builtin_fmaf(a2, ml[j][1], L2);
                o1 += a1 * pj[j];
                o2 += a2 * pj[j];
            }
            if (xs_role == 1) {  // block p is B's alone: final rows
                const int rowp = 32 * xs_p + qi;
                if (rowp < S) store_o(reinterpret_cast<floatx4 *>(obase + (size_t)rowp * ors + 4 * ch), o2 * __builtin_amdgcn_rcpf(L2));
            }
            const int row = 32 * (xs_role == 2 ? qblk : xs_q) + qi;
            if (xs_role == 2) {
                if (row < S) store_o(reinterpret_cast<floatx4 *>(obase + (size_t)row * ors + 4 * ch), o1 * __builtin_amdgcn_rcpf(L1));
                return;
            }
            float *mine = reinterpret_cast<float *>(slots + (2 * pg + xs_role) * SLOT);
            const float *other = reinterpret_cast<const float *>(slots + (2 * pg + (xs_role ^ 1)) * SLOT);
            bool merge = (xw[0] & 1u) != 0;
            if (merge) {
                if (tid == 0) __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                store_agent(mine + qi * D + 4 * ch, o1);
                if (ch == 0) store_agent(mine + 32 * D + 2 * qi, float2v{M1, L1});
                wait_vm_barrier<0>();  // every wave's part of the partial is stored
                if (tid == 0) xw[1] = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                wait_vm_barrier<0>();
                merge = (xw[1] & 1u) != 0;
            }
            if (merge) {
                floatx4 op;
                float2v mp;
                load_agent(other + qi * D + 4 * ch, other + 32 * D + 2 * qi, op, mp);
                // Combined in the fixed order (A's partial, B's partial) whichever workgroup merges,
                // so the result does not depend on which one arrived last.
                const bool am_a = xs_role == 0;
                const floatx4 oa = am_a ? o1 : op, ob = am_a ? op : o1;
                const float ma = am_a ? M1 : mp[0], mb = am_a ? mp[0] : M1;
                const float la = am_a ? L1 : mp[1], lb = am_a ? mp[1] : L1;
                const float mx = fmaxf(ma, mb);
                const float wa = __builtin_amdgcn_exp2f(ma - mx), wb = __builtin_amdgcn_exp2f(mb - mx);
                const floatx4 res = (wa * oa + wb * ob) * __builtin_amdgcn_rcpf(__builtin_fmaf(wa, la, wb * lb));
                if (row < S) store_o(reinterpret_cast<floatx4 *>(obase + (size_t)row * ors + 4 * ch), res);
            }
            return;
        }
        wait_vm_barrier<0>();
        if constexpr (DC == 16 && NS == 8 && C::BM * DC == C::NT) {
            // One thread per (query, 4 columns): a query's 16 threads are one 16-lane DPP row. Lanes
            // j and j+8 of the row read split j's (m, l); the row's max M and L = sum_j w_j l_j
            // (w_j = exp2(m_j - M)) come from three DPP steps each, and lane j's normalised weight
            // w_j / L is broadcast to the row once per split (row_newbcast), so each thread forms
            // one exponential instead of eight. The reductions use commutative pairings only, so
            // every lane of a row holds bitwise the same M and L.
            const int qi = tid >> 4, ch = tid & 15;
            floatx4 pj[NS];  // read first, so the LDS reads overlap the weights' DPP chain
#pragma unroll
            for (int j = 0; j < NS; ++j) pj[j] = *part(j, qi, ch);
            const float2v mlj = mlb[qi * NS + (ch & 7)];
            float mx = mlj[0];
            mx = fmaxf(mx, dpp_f32<0xB1>(mx));   // quad_perm [1,0,3,2]
            mx = fmaxf(mx, dpp_f32<0x4E>(mx));   // quad_perm [2,3,0,1]
            mx = fmaxf(mx, dpp_f32<0x141>(mx));  // row_half_mirror: the two quads of each half-row
            const float wj = __builtin_amdgcn_exp2f(mlj[0] - mx);  // 0 for a split that saw no key
            float den = wj * mlj[1];
            den += dpp_f32<0xB1>(den);
            den += dpp_f32<0x4E>(den);
            den += dpp_f32<0x141>(den);
            const float wn = wj * __builtin_amdgcn_rcpf(den);
            // the partial reads complete here, not later inside the store's row test
            asm volatile("" ::"v"(wn), "v"(pj[0]), "v"(pj[1]), "v"(pj[2]), "v"(pj[3]), "v"(pj[4]), "v"(pj[5]),
                         "v"(pj[6]), "v"(pj[7]));
            floatx4 res = dpp_f32<0x150>(wn) * pj[0];  // row_newbcast:0
            static_for<1, NS>([&](auto jc) {
                constexpr int J = decltype(jc)::value;
                res += dpp_f32<0x150 + J>(wn) * pj[J];  // row_newbcast:J
            });
            const int row = q0 + qi;
            if (row < S) store_o(reinterpret_cast<floatx4 *>(obase + (size_t)row * ors + 4 * ch), res);
            NC_TL_END()
            return;
        }
        for (int u = tid; u < C::BM * DC; u += C::NT) {
            const int qi = u / DC, ch = u % DC;
            const int row = q0 + qi;
            if (row >= S) continue;
            float2v ml[NS];
            floatx4 pj[NS];
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                ml[j] = mlb[qi * NS + j];
                pj[j] = *part(j, qi, ch);
            }
            float mmax = ml[0][0];
#pragma unroll
            for (int j = 1; j < NS; ++j) mmax = fmaxf(mmax, ml[j][0]);
            float den = 0.f;
            floatx4 res = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                const float wj = __builtin_amdgcn_exp2f(ml[j][0] - mmax);  // exp2(-inf) = 0
                den = __builtin_fmaf(wj, ml[j][1], den);
                res += wj * pj[j];
            }
            store_o(reinterpret_cast<floatx4 *>(obase + (size_t)row * ors + 4 * ch), res * __builtin_amdgcn_rcpf(den));
        }
        NC_TL_END()
        return;
    }

    // Epilogue, shared staging. (1) Each wave publishes its per-query (m, l) in a dedicated LDS
    // area (other waves may still read the ring). (2) After one barrier every lane derives, for
    // its query, the merge weight exp2(m_s - M) / L of its own partial (M = max over the NS key
    // splits, L = sum exp2(m_j - M) l_j), scales its O^T partial in registers and writes it over
    // the ring. (3) After a second barrier each output float4 is the plain sum of NS scaled
    // partials, stored row-contiguously (coalesced). With NS = 1 the weight is 1 / l.
    if (hh == 0) mlb[(qg * 32 + c) * NS + s] = float2v{mrow, lt};
    wait_vm_barrier<0>();
    float scale_own;
    if constexpr (NS == 1) {
        scale_own = __builtin_amdgcn_rcpf(lt);
    } else {
        const float2v *row = mlb + (qg * 32 + c) * NS;
        float2v ml[NS];
#pragma unroll
        for (int j = 0; j < NS; ++j) ml[j] = row[j];
        float mmax = ml[0][0];
#pragma unroll
        for (int j = 1; j < NS; ++j) mmax = fmaxf(mmax, ml[j][0]);
        float den = 0.f;
#pragma unroll
        for (int j = 0; j < NS; ++j) den = __builtin_fmaf(__builtin_amdgcn_exp2f(ml[j][0] - mmax), ml[j][1], den);
        scale_own = __builtin_amdgcn_exp2f(mrow - mmax) * __builtin_amdgcn_rcpf(den);  // 0 for empty splits
    }
    // 32-bit LDS pointers: with generic ones the compiler keeps 64-bit address parts live across
    // the key loop of these register-tight kernels.
    NC_LDS(float) *ob = reinterpret_cast<NC_LDS(float) *>((uintptr_t)lds0);
    {
        NC_LDS(float) *dst = ob + (w * 32 + c) * C::OP;
#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = 32 * mt + 8 * i + 4 * hh;
                if (d < D) {
                    floatx4 t = {o[mt][4 * i], o[mt][4 * i + 1], o[mt][4 * i + 2], o[mt][4 * i + 3]};
                    *reinterpret_cast<NC_LDS(floatx4) *>(dst + d) = t * scale_own;
                }
            }
    }
    __syncthreads();
    for (int u = tid; u < C::BM * DC; u += C::NT) {
        const int qi = u / DC, ch = u % DC;
        const int row = q0 + qi;
        if (row >= S) continue;
        const NC_LDS(float) *src = ob + ((qi / 32) * NS * 32 + (qi % 32)) * C::OP + 4 * ch;
        floatx4 parts[NS];
#pragma unroll
        for (int j = 0; j < NS; ++j) parts[j] = *reinterpret_cast<const NC_LDS(floatx4) *>(src + 32 * j * C::OP);
        floatx4 res = parts[0];
#pragma unroll
        for (int j = 1; j < NS; ++j) res += parts[j];
        store_o(reinterpret_cast<floatx4 *>(obase + (size_t)row * ors + 4 * ch), res);
    }
    NC_TL_END()
}

// A dispatched pipelined kernel: its LDS, and launch index blockIdx.x mapped by pipe_slot.
template <int D, int NQ, int NS, bool CAUSAL, int NSTAGE, int SUB, bool BF, bool XS = false>
__device__ __forceinline__ void flash_fwd_pipe_kernel(const nc_flash_kernel_args &a) {
    __shared__ __attribute__((aligned(16))) char smem[pipe_lds_bytes<D, NQ, NS, NSTAGE, SUB, XS>()];
    flash_fwd_pipe_body<D, NQ, NS, CAUSAL, NSTAGE, SUB, BF, XS>(a, smem, [](uint32_t bh) { return pipe_slot(blockIdx.x, bh); });
}

// Dense-layout form of the private-staging kernels (the `d` kernels, e.g. q1s8p2d), for launches whose four
// tensors are packed slices (slice stride seq_len*D elements, row stride D). The argument block is
// the same nc_flash_kernel_args, declared as one kernel parameter per field so that the code object
// asks for its first seven (q, k, v, o, seq_len, head_dim, q_stride: 14 SGPRs) to be preloaded into
// SGPRs at wave launch; with the layout implied by seq_len and D, and the workgroup's slot taken
// from its 3-D workgroup id, a wave reaches its first Q and K/V loads without waiting for any
// memory. The other fields are read where they are needed (scale in the softmax, off the path to
// the first loads). Grid (8, batch_heads/8, nqb) when batch_heads is a multiple of 8, else
// (batch_heads, 1, nqb): workgroups are dealt to the XCDs in linear order, so with 8 in x each XCD
// takes the heads x, x+8, ... (their K/V in its L2), and z runs from the heaviest causal block.
template <int D, int NS, bool CAUSAL, int NSTAGE, bool BF>
__device__ __forceinline__ void flash_fwd_dense_kernel(const uint16_t *q, const uint16_t *k, const uint16_t *v, float *o,
                                                       uint64_t seq_len, uint64_t head_dim, float scale, void *scratch) {
    __shared__ __attribute__((aligned(16))) char smem[pipe_lds_bytes<D, 1, NS, NSTAGE, 1, false>()];
    nc_flash_kernel_args a;
    const uint64_t slice = seq_len * D;
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = o;
    a.seq_len = seq_len;
    a.head_dim = head_dim;
    a.q_stride = a.k_stride = a.v_stride = a.o_stride = slice;
    a.scale = scale;
    a.causal = CAUSAL ? 1u : 0u;
    a.q_row_stride = a.k_row_stride = a.v_row_stride = a.o_row_stride = D;
    a.batch_heads = 0;  // the slot comes from the workgroup id
    a.num_q_blocks = (uint32_t)((seq_len + 31) / 32);
    a.scratch = scratch;  // unused by these kernels but for the timeline code object's stamps
    a.balance_tail = 0;
    flash_fwd_pipe_body<D, 1, NS, CAUSAL, NSTAGE, 1, BF>(a, smem, [](uint32_t) {
        const uint32_t L = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);  // timeline stamps only
        return PipeSlot{L, blockIdx.x + 8u * blockIdx.y, blockIdx.z};
    });
}

// ---------------------------------------------------------------------------------------------
// Reference-ABI entry points: the kernel symbols the reference's code object exports
// (flash_attention_fwd_{v2,opt,h64,h64_bn32,h64_causal} and the legacy flash_attention_fwd,
// src/main_device.zig:19-47) with their parameter list (q, k, v, o, seq_len, head_dim,
// q/k/v/o_stride, scale, causal; 88 bytes) and launch geometry: grid (ceil(S/16), batch_heads),
// block = the reference's thread count (64 or 128: one or two waves), rows of exactly head_dim
// elements, any slice stride and base alignment. They exist so callers that look kernels up by
// the reference's names (src/main.zig:822-828, 1024-1030) keep working; nc_flash_launch with the
// gfx950 dispatch is the fast path.
//
// Workgroup (bx, by): query rows 16bx .. 16bx+15 of slice by. Every wave computes those 16 rows
// over every NW-th 32-key chunk with 16x16x32 MFMAs in the transposed form (S^T = K Q^T,
// O^T += V^T P^T); with 16-byte aligned slices each wave stages its chunks of K and V through its
// own LDS region, otherwise operands are gathered element by element from global memory (no
// alignment assumed); the softmax takes each chunk's max after scaling (any sign of scale), and the
// waves' partials merge through LDS. Lane l holds query l%16; in S^T tile t it holds keys 16t+4(l/16)+r,
// and those 8 keys are, in order, its k-values of the P^T and V^T operands.
// ---------------------------------------------------------------------------------------------
// LDS of the reference-ABI body: WAVES staging regions, each one staged 32-key chunk of K and of V
// (rows padded to D + 8 halves: the K reads of 16 rows at one column chunk and the transposed V
// reads then spread over the banks), reused after the key loop for the waves' merge. A launch of
// NW waves runs two chunk streams per wave when 2 NW regions exist, else one (NW regions).
template <int D, int WAVES>
struct RefCfg {
    static constexpr int KP = D + 8;                 // staged row pitch, halves
    static constexpr int CHUNK = 32 * KP * 2;        // bytes of one staged K (or V) chunk
    static constexpr int WAVE = 2 * CHUNK;
    static constexpr int OP = D + 4;                 // merge row pitch, floats
    static constexpr int MERGE = WAVES * 16 * (8 + OP * 4);
    static constexpr int LDS = WAVES * WAVE > MERGE ? WAVES * WAVE : MERGE;
    static constexpr int SEG = 32 * (D / 8) / 64;    // 16-byte segments of a chunk per lane
};
// A symbol's LDS (d = 64 needs the most). The symbols the reference launches with 128 threads
// hold four regions (two waves, two streams each); those it launches with 64 threads hold two (one
// wave, two streams), so eight of their one-wave workgroups fit a CU instead of four, and accept at
// most two waves.
template <int WAVES>
constexpr int ref_lds_bytes() { return RefCfg<64, WAVES>::LDS; }
// A symbol's LDS: its staging regions, or what the pipelined forms it may run need (the 128-thread
// symbols: 32 rows over two key-split waves, or 64 rows over two query waves; the 64-thread ones:
// 32 rows on one wave), whichever is more.
template <int WAVES>
constexpr int ref_symbol_lds_bytes() {
    constexpr int pipe = WAVES >= 4 ? (pipe_lds_bytes<64, 1, 2, 2, 1, false>() > pipe_lds_bytes<64, 2, 1, 2, 2, false>()
                                           ? pipe_lds_bytes<64, 1, 2, 2, 1, false>()
                                           : pipe_lds_bytes<64, 2, 1, 2, 2, false>())
                                    : pipe_lds_bytes<64, 1, 1, 2, 1, false>();
    return ref_lds_bytes<WAVES>() > pipe ? ref_lds_bytes<WAVES>() : pipe;
}
// Grid size (workgroups) from which the 128-thread d=64 launches take four 16-row blocks per
// working workgroup instead of two (flash_fwd_refabi). Measured on MI355X with the reference's
// grid: the four-block form is 5.5 % faster on c5 (32768 workgroups: the L2 traffic binds), equal
// on c4 (8192), and 10-37 % slower from 1536 to 4096 workgroups.
#ifndef NC_REF_COARSE_MIN_WORKGROUPS
#define NC_REF_COARSE_MIN_WORKGROUPS 16384
#endif
constexpr uint64_t kRefCoarseMinWorkgroups = NC_REF_COARSE_MIN_WORKGROUPS;


// VEC: every Q/K/V slice base is 16-byte aligned (pointers and slice strides; rows of D halves
// are), so each wave loads a key chunk as one contiguous run of 16-byte segments, stages it in its
// own LDS region (the next chunk's loads in flight meanwhile) and reads the MFMA operands there:
// K rows by ds_read_b128, V^T by ds_read_b64_tr_b16 (lane m of a 16-lane group supplies
// V[r0 + m/4][d0 + 4(m%4)], lane i receives V[r0..r0+3][d0 + i]). Otherwise every operand element
// is gathered from global memory (any stride, any base alignment).
template <int D, bool VEC, int WAVES>
__device__ __forceinline__ void flash_fwd_refabi_body(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                                      float *o, int S, uint64_t q_stride, uint64_t k_stride,
                                                      uint64_t v_stride, uint64_t o_stride, float scale,
                                                      bool causal, char *smem) {
    using RC = RefCfg<D, WAVES>;
    constexpr int DH = (D + 31) / 32;  // 32-column k-steps of S^T
    constexpr int DT = D / 16;         // 16-row O^T tiles
    constexpr int OP = RC::OP;
    const int NW = (int)(blockDim.x >> 6);
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
    // Causal: the last (heaviest) query blocks first, so that on grids larger than the machine
    // holds at once they do not start last.
    const int r0 = 16 * (int)(causal ? gridDim.x - 1u - blockIdx.x : blockIdx.x);
    const size_t head = blockIdx.y;
    if (r0 >= S) return;
    const uint16_t *qh = q + head * q_stride, *kh = k + head * k_stride, *vh = v + head * v_stride;
    float *oh = o + head * o_stride;
    const int qrow = r0 + c;
    const int lim_row = causal ? min(qrow, S - 1) : S - 1;  // last key visible to this lane's query
    const int kv_end = causal ? min(S, r0 + 16) : S;
    const int nch = (kv_end + 31) >> 5;

    auto gather8 = [&](const uint16_t *base, int row, int d0) {  // 8 f16 of one row, zero outside
        half8 x = {};
        if (row < S) {
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (d0 + j < D) x[j] = __builtin_bit_cast(_Float16, base[(size_t)row * D + d0 + j]);
        }
        return x;
    };
    auto load8 = [&](const uint16_t *base, int row, int d0) {  // the same by one 16-byte load
        u32x4 t = {0u, 0u, 0u, 0u};
        if (row < S && d0 < D) t = *reinterpret_cast<const u32x4 *>(base + (size_t)row * D + d0);
        return __builtin_bit_cast(half8, t);
    };
    half8 qf[DH];
#pragma unroll
    for (int h = 0; h < DH; ++h) qf[h] = VEC ? load8(qh, qrow, 32 * h + 8 * g) : gather8(qh, qrow, 32 * h + 8 * g);

    // This wave's staging region (VEC): K rows at kst, V rows at kst + CHUNK, pitch KP halves.
    // This wave's staging region (VEC): K rows at kst, V rows at kst + CHUNK, pitch KP halves; the
    // next chunk's rows travel in registers while the current one is computed (deeper register
    // prefetch measured no faster).
    const uint32_t kst = (uint32_t)(uintptr_t)smem + w * RC::WAVE;
    const uint32_t vst = kst + RC::CHUNK;
    u32x4 kreg[RC::SEG > 0 ? RC::SEG : 1], vreg[RC::SEG > 0 ? RC::SEG : 1];
    auto fetch = [&](int ch) {  // chunk ch's K and V rows into registers, zero past seq_len
#pragma unroll
        for (int j = 0; j < RC::SEG; ++j) {
            const int seg = lane + 64 * j, row = seg / (D / 8), c8 = seg % (D / 8), key = 32 * ch + row;
            const u32x4 z = {0u, 0u, 0u, 0u};
            kreg[j] = key < S ? *reinterpret_cast<const u32x4 *>(kh + (size_t)key * D + 8 * c8) : z;
            vreg[j] = key < S ? *reinterpret_cast<const u32x4 *>(vh + (size_t)key * D + 8 * c8) : z;
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int j = 0; j < RC::SEG; ++j) {
            const int seg = lane + 64 * j, row = seg / (D / 8), c8 = seg % (D / 8);
            const uint32_t off = (uint32_t)(row * RC::KP + 8 * c8) * 2;
            *reinterpret_cast<NC_LDS(u32x4) *>((uintptr_t)(kst + off)) = kreg[j];
            *reinterpret_cast<NC_LDS(u32x4) *>((uintptr_t)(vst + off)) = vreg[j];
        }
    };
    // Two chunk streams per wave (VEC, two staging regions per wave: the reference's 64- and
    // 128-thread launches, on slices that fit 32-bit buffer offsets). One wave per SIMD has nothing else to hide
    // a chunk's serial chain of LDS round trips, MFMAs and cross-lane reductions, so each wave keeps
    // two online-softmax states, A over its chunks w, w + 2NW, ... and B over w + NW, w + 3NW, ...,
    // runs the two chains side by side in one branch-free body and merges them after the loop. Each
    // stream stages in its own region (the two regions of a wave are the ones two more waves would
    // use), and the next pair's rows are fetched by range-checked buffer loads, which read zero past
    // the slice.
    const bool pair = VEC && 2 * NW <= WAVES && (uint64_t)S * D * 2 < (1ull << 31);
    if (VEC && !pair && w < nch) fetch(w);

    const float sc = scale * kLog2e;
    float mrow = neg_inf(), l = 0.f;
    floatx4 oacc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[dt] = floatx4{};
    const half2v ones = {(_Float16)1.0f, (_Float16)1.0f};

    if constexpr (VEC) {
        if (pair) {
            const uint32_t span = (uint32_t)S * D * 2;
            const __amdgpu_buffer_rsrc_t krs = make_rsrc(kh, span), vrs = make_rsrc(vh, span);
            const uint32_t kA = (uint32_t)(uintptr_t)smem + 2 * w * RC::WAVE, kB = kA + RC::WAVE;
            u32x4 kra[RC::SEG], vra[RC::SEG], krb[RC::SEG], vrb[RC::SEG];
            auto fetch2 = [&](int ch, u32x4(&kr)[RC::SEG], u32x4(&vr)[RC::SEG]) {
#pragma unroll
                for (int j = 0; j < RC::SEG; ++j) {
                    const int seg = lane + 64 * j, row = seg / (D / 8), c8 = seg % (D / 8);
                    const uint32_t off = (uint32_t)((32 * ch + row) * D + 8 * c8) * 2;
                    kr[j] = __builtin_amdgcn_raw_buffer_load_b128(krs, off, 0, 0);
                    vr[j] = __builtin_amdgcn_raw_buffer_load_b128(vrs, off, 0, 0);
                }
            };
            auto stage2 = [&](uint32_t kst2, const u32x4(&kr)[RC::SEG], const u32x4(&vr)[RC::SEG]) {
#pragma unroll
                for (int j = 0; j < RC::SEG; ++j) {
                    const int seg = lane + 64 * j, row = seg / (D / 8), c8 = seg % (D / 8);
                    const uint32_t off = (uint32_t)(row * RC::KP + 8 * c8) * 2;
                    *reinterpret_cast<NC_LDS(u32x4) *>((uintptr_t)(kst2 + off)) = kr[j];
                    *reinterpret_cast<NC_LDS(u32x4) *>((uintptr_t)(kst2 + RC::CHUNK + off)) = vr[j];
                }
            };
            auto scores = [&](uint32_t kst2, floatx4(&s)[2]) {
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    s[t] = floatx4{};
#pragma unroll
                    for (int h = 0; h < DH; ++h) {
                        const int d0 = 32 * h + 8 * g;
                        half8 kf = half8{};
                        if (d0 < D)
                            kf = *reinterpret_cast<const NC_LDS(half8) *>(
                                (uintptr_t)(kst2 + (uint32_t)((16 * t + c) * RC::KP + d0) * 2));
                        s[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[h], s[t], 0, 0, 0);
                    }
                }
            };
            auto vtread = [&](uint32_t vst2, u32x2(&vt)[2 * DT]) {
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                    for (int hf = 0; hf < 2; ++hf) {
                        const int r = 16 * hf + 4 * g + (c >> 2), d0 = 16 * dt + 4 * (c & 3);
                        ds_read_tr<0>(vt[2 * dt + hf], vst2 + (uint32_t)(r * RC::KP + d0) * 2);
                    }
            };
            // Online softmax of one chunk into one stream's (m, l, O), returning P (f16).
            auto softmax = [&](const floatx4(&s)[2], int kt0, float &m, float &lsum, floatx4(&oa)[DT]) {
                float x[8];
                float lm = neg_inf();
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int key = kt0 + 16 * (e >> 2) + 4 * g + (e & 3);
                    x[e] = key > lim_row ? neg_inf() : s[e >> 2][e & 3] * sc;
                    lm = fmaxf(lm, x[e]);
                }
                lm = fmaxf(lm, __shfl_xor(lm, 16));
                lm = fmaxf(lm, __shfl_xor(lm, 32));
                const float m_new = fmaxf(m, lm);
                const float m_use = m_new == neg_inf() ? 0.f : m_new;
                const float alpha = __builtin_amdgcn_exp2f(m - m_use);
                lsum *= alpha;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) oa[dt] *= alpha;
                m = m_new;
                half8 pb;
#pragma unroll
                for (int e = 0; e < 8; ++e) pb[e] = (_Float16)__builtin_amdgcn_exp2f(x[e] - m_use);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const half2v hp = {pb[2 * t], pb[2 * t + 1]};
                    lsum = __builtin_amdgcn_fdot2(hp, ones, lsum, false);
                }
                return pb;
            };
            auto pv = [&](const u32x2(&vt)[2 * DT], const half8 &pb, floatx4(&oa)[DT]) {
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    const u32x4 vv = {vt[2 * dt][0], vt[2 * dt][1], vt[2 * dt + 1][0], vt[2 * dt + 1][1]};
                    oa[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, vv), pb, oa[dt], 0, 0, 0);
                }
            };
            float m1 = neg_inf(), l1 = 0.f;
            floatx4 o1[DT];
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o1[dt] = floatx4{};
            fetch2(w, kra, vra);
            fetch2(w + NW, krb, vrb);
            int ch = w;
            for (; ch + NW < nch; ch += 2 * NW) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // both regions' previous reads are done
                stage2(kA, kra, vra);
                stage2(kB, krb, vrb);
                asm volatile("" ::: "memory");
                fetch2(ch + 2 * NW, kra, vra);  // in flight while this pair is computed
                fetch2(ch + 3 * NW, krb, vrb);
                floatx4 sa[2], sb[2];
                scores(kA, sa);
                scores(kB, sb);
                u32x2 vta[2 * DT], vtb[2 * DT];
                vtread(kA + RC::CHUNK, vta);
                vtread(kB + RC::CHUNK, vtb);
                const half8 pa = softmax(sa, 32 * ch, mrow, l, oacc);
                const half8 pbb = softmax(sb, 32 * (ch + NW), m1, l1, o1);
                pv(vta, pa, oacc);
                pv(vtb, pbb, o1);
            }
            if (ch < nch) {  // an odd last chunk: stream A alone (its registers hold chunk ch)
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                stage2(kA, kra, vra);
                asm volatile("" ::: "memory");
                floatx4 sa[2];
                scores(kA, sa);
                u32x2 vta[2 * DT];
                vtread(kA + RC::CHUNK, vta);
                const half8 pa = softmax(sa, 32 * ch, mrow, l, oacc);
                pv(vta, pa, oacc);
            }
            // Stream B into A (row-uniform maxima; a stream that saw no chunk has m = -inf, l = O = 0).
            const float mm = fmaxf(mrow, m1);
            const float mu = mm == neg_inf() ? 0.f : mm;
            const float a0 = __builtin_amdgcn_exp2f(mrow - mu), a1 = __builtin_amdgcn_exp2f(m1 - mu);
            l = l * a0 + l1 * a1;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) oacc[dt] = oacc[dt] * a0 + o1[dt] * a1;
            mrow = mm;
        }
    }

    for (int ch = w; !pair && ch < nch; ch += NW) {
        const int kt0 = 32 * ch;
        if constexpr (VEC) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the previous chunk's reads are done
            stage();
            asm volatile("" ::: "memory");
            if (ch + NW < nch) fetch(ch + NW);  // in flight while this chunk is computed
        }
        floatx4 s[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            s[t] = floatx4{};
#pragma unroll
            for (int h = 0; h < DH; ++h) {
                half8 kf;
                if constexpr (VEC) {
                    const int d0 = 32 * h + 8 * g;
                    kf = half8{};
                    if (d0 < D)
                        kf = *reinterpret_cast<const NC_LDS(half8) *>((uintptr_t)(kst + (uint32_t)((16 * t + c) * RC::KP + d0) * 2));
                } else {
                    kf = gather8(kh, kt0 + 16 * t + c, 32 * h + 8 * g);
                }
                s[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[h], s[t], 0, 0, 0);
            }
        }
        // V^T operands (VEC): issued now, their latency hidden behind the softmax.
        u32x2 vt[VEC ? 2 * DT : 1];
        if constexpr (VEC) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    const int r = 16 * hf + 4 * g + (c >> 2), d0 = 16 * dt + 4 * (c & 3);
                    ds_read_tr<0>(vt[2 * dt + hf], vst + (uint32_t)(r * RC::KP + d0) * 2);
                }
        }
        float x[8];
        float lm = neg_inf();
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int key = kt0 + 16 * (e >> 2) + 4 * g + (e & 3);
            x[e] = key > lim_row ? neg_inf() : s[e >> 2][e & 3] * sc;
            lm = fmaxf(lm, x[e]);
        }
        lm = fmaxf(lm, __shfl_xor(lm, 16));
        lm = fmaxf(lm, __shfl_xor(lm, 32));
        const float m_new = fmaxf(mrow, lm);
        const float m_use = m_new == neg_inf() ? 0.f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(mrow - m_use);
        l *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
        mrow = m_new;
        half8 pb;
#pragma unroll
        for (int e = 0; e < 8; ++e) pb[e] = (_Float16)__builtin_amdgcn_exp2f(x[e] - m_use);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const half2v hp = {pb[2 * t], pb[2 * t + 1]};
            l = __builtin_amdgcn_fdot2(hp, ones, l, false);
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            half8 va;
            if constexpr (VEC) {
                const u32x4 vv = {vt[2 * dt][0], vt[2 * dt][1], vt[2 * dt + 1][0], vt[2 * dt + 1][1]};
                va = __builtin_bit_cast(half8, vv);
            } else {
                va = half8{};
                const int d = 16 * dt + c;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int key = kt0 + 16 * (e >> 2) + 4 * g + (e & 3);
                    if (key < S) va[e] = __builtin_bit_cast(_Float16, vh[(size_t)key * D + d]);
                }
            }
            oacc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb, oacc[dt], 0, 0, 0);
        }
    }

    // Merge the waves' partials: per-query (m, l) and scaled O^T through LDS (over the staging
    // regions, once every wave is past its loop).
    float lt = l + __shfl_xor(l, 16);
    lt += __shfl_xor(lt, 32);
    __syncthreads();
    float2v *mlb = reinterpret_cast<float2v *>(smem);                                  // [NW][16]
    float *ob = reinterpret_cast<float *>(smem + WAVES * 16 * sizeof(float2v));  // [NW][16][OP]
    if (g == 0) mlb[w * 16 + c] = float2v{mrow, lt};
    __syncthreads();
    float mmax = neg_inf(), den = 0.f;
    for (int j = 0; j < NW; ++j) mmax = fmaxf(mmax, mlb[j * 16 + c][0]);
    for (int j = 0; j < NW; ++j) den += __builtin_amdgcn_exp2f(mlb[j * 16 + c][0] - mmax) * mlb[j * 16 + c][1];
    const float wgt = __builtin_amdgcn_exp2f(mrow - mmax) / den;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) ob[(w * 16 + c) * OP + 16 * dt + 4 * g + r] = oacc[dt][r] * wgt;
    __syncthreads();
    for (int u = threadIdx.x; u < 16 * D; u += blockDim.x) {
        const int qi = u / D, d = u % D;
        if (r0 + qi >= S) continue;
        float acc = 0.f;
        for (int j = 0; j < NW; ++j) acc += ob[(j * 16 + qi) * OP + d];
        oh[(size_t)(r0 + qi) * D + d] = acc;
    }
}

// The per-symbol contract of the reference's kernels:
//   ALWAYS_CAUSAL  the causal argument is ignored and the mask always applies
//                  (flash_attention_fwd_h64_causal: `_ = causal`, src/flash_h64_causal.zig:34, and the
//                  unconditional key_row <= q_row test of :113-118);
//   D64_ONLY       head_dim != 64 returns without writing (src/flash_h64.zig:35,
//                  src/flash_h64_bn32.zig:40, src/flash_h64_causal.zig:35); the other symbols accept
//                  head_dim 16, 32 and 64 (src/flash_v2.zig:37, src/flash_opt.zig:31, src/kernels.zig:394).
template <bool ALWAYS_CAUSAL, bool D64_ONLY, int WAVES>
__device__ __forceinline__ void flash_fwd_refabi(const uint16_t *q, const uint16_t *k, const uint16_t *v, float *o,
                                                 uint64_t seq_len, uint64_t head_dim, uint64_t q_stride,
                                                 uint64_t k_stride, uint64_t v_stride, uint64_t o_stride, float scale,
                                                 uint32_t causal) {
    __shared__ __attribute__((aligned(16))) char smem[ref_symbol_lds_bytes<WAVES>()];
    // Shapes the reference's kernels reject return without writing (src/flash_h64_bn32.zig:40), and
    // launches of more waves than the symbol's LDS stages.
    if (seq_len == 0 || seq_len > 0x7fffffffull || (blockDim.x & 63) || blockDim.x > 64u * WAVES) return;
    const int S = (int)seq_len;
    const bool cz = ALWAYS_CAUSAL || causal != 0;
    // 16-byte vector path when every slice base is 16-byte aligned (rows of head_dim halves are).
    const bool vec = ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                       reinterpret_cast<uintptr_t>(v)) & 15u) == 0 && ((q_stride | k_stride | v_stride) & 7u) == 0;
    auto run = [&](auto dc, auto vc) {
        flash_fwd_refabi_body<decltype(dc)::value, decltype(vc)::value != 0, WAVES>(q, k, v, o, S, q_stride, k_stride,
                                                                                     v_stride, o_stride, scale, cz, smem);
    };
    // The pipelined body for `nqb` row blocks of BM rows: its argument block (rows of head_dim
    // elements; no scratch, no balancing) and slot (block m of slice blockIdx.y; causal blocks come
    // heaviest first, as in the 16-row body, since qb_rev counts from the last block).
    auto pipe_run = [&](auto dc, auto nq_c, auto ns_c, auto sub_c, uint32_t m) {
        constexpr int DD = decltype(dc)::value, NQ = decltype(nq_c)::value, NS = decltype(ns_c)::value;
        constexpr int SUB = decltype(sub_c)::value;
        nc_flash_kernel_args a = {};
        a.q = q;
        a.k = k;
        a.v = v;
        a.o = o;
        a.seq_len = seq_len;
        a.head_dim = DD;
        a.q_stride = q_stride;
        a.k_stride = k_stride;
        a.v_stride = v_stride;
        a.o_stride = o_stride;
        a.scale = scale;
        a.causal = cz ? 1u : 0u;
        a.q_row_stride = a.k_row_stride = a.v_row_stride = a.o_row_stride = DD;
        a.batch_heads = gridDim.y;
        a.num_q_blocks = (uint32_t)((seq_len + 32 * NQ - 1) / (32 * NQ));
        const uint32_t head = blockIdx.y;
        auto slot = [&](uint32_t) { return PipeSlot{0u, head, m}; };
        if (cz)
            flash_fwd_pipe_body<DD, NQ, NS, true, 2, SUB, false>(a, smem, slot);
        else
            flash_fwd_pipe_body<DD, NQ, NS, false, 2, SUB, false>(a, smem, slot);
    };
    // Layout the pipelined body needs: 16-byte aligned Q/K/V slices, float4-aligned O slices (its O
    // stores), slices within its 32-bit buffer offsets (up to one block past seq_len), and a grid of
    // exactly ceil(S/16) blocks per slice, so that no row outside the launch is written.
    const bool o_vec = (reinterpret_cast<uintptr_t>(o) & 15u) == 0 && (o_stride & 3u) == 0;
    const bool pipe_ok = vec && o_vec && (seq_len + 512) * head_dim * 2 < (1ull << 31) &&
                         gridDim.x == (seq_len + 15) / 16;
    // Very large d=64 grids of two-wave workgroups (the reference's 128-thread launches): one
    // workgroup of each group of four consecutive 16-row blocks computes the group's 64 rows with
    // the pipelined body (two 32-row query waves sharing each staged K/V block), and the other three
    // return. Each K/V byte staged then serves 64 queries instead of 16. Which workgroup of a group
    // works rotates with the group and the slice, so the working ones spread over the XCDs.
    constexpr bool COARSE = WAVES >= 4;  // the two-wave pipelined forms (their LDS: ref_symbol_lds_bytes)
    if (COARSE && pipe_ok && head_dim == 64 && blockDim.x == 128 &&
        (uint64_t)gridDim.x * gridDim.y >= kRefCoarseMinWorkgroups) {
        const uint32_t gx = gridDim.x, bx = blockIdx.x, by = blockIdx.y, m = bx >> 2;
        const uint32_t sz = gx - 4u * m < 4u ? gx - 4u * m : 4u;
        if (bx == 4u * m + (by + m) % sz) pipe_run(IC<64>{}, IC<2>{}, IC<1>{}, IC<2>{}, m);
        return;
    }
    // One-wave workgroups (the reference's 64-thread launches): one workgroup of each pair of
    // consecutive 16-row blocks computes both with the pipelined body (one 32-row wave, private
    // two-stage staging), the other returns; the working one alternates with the pair and the slice.
    // Measured on MI355X against the 16-row body with the reference's grid: 1.5-2.2x faster from
    // 1024 workgroups, 3-27 % faster on smaller grids, but 2-7 % slower on causal launches over few
    // slices and long sequences (d=32 BH=2-4, S=1024-2048: half the waves then carry the heavy
    // blocks), which keep the 16-row body.
    const bool pair_coarse = pipe_ok && blockDim.x == 64 &&
                             (!cz || gridDim.y >= 8 || (uint64_t)gridDim.x * gridDim.y >= 512);
    auto run_pairs = [&](auto dc) {
        static_assert(pipe_lds_bytes<decltype(dc)::value, 1, 1, 2, 1, false>() <= ref_symbol_lds_bytes<2>(),
                      "the pipelined body fits the LDS");
        const uint32_t gx = gridDim.x, bx = blockIdx.x, by = blockIdx.y, m = bx >> 1;
        const uint32_t sz = gx - 2u * m < 2u ? gx - 2u * m : 2u;
        if (bx == 2u * m + (by + m) % sz) pipe_run(dc, IC<1>{}, IC<1>{}, IC<1>{}, m);
    };
    // Two-wave workgroups below the four-block form's grid size: one workgroup of each pair of
    // 16-row blocks computes both (32 rows) with the pipelined body, its two waves splitting the
    // keys. Measured on MI355X against the 16-row body with the reference's grid: 10-44 % faster on
    // every shape tried (c3 14.6 -> 12.5 us, c1 3.16 -> 2.68 us, d=64 BH=4 S=4096 causal 57 -> 32 us).
    const bool pair2 = COARSE && pipe_ok && blockDim.x == 128;
    auto run_pairs2 = [&](auto dc) {
        const uint32_t gx = gridDim.x, bx = blockIdx.x, by = blockIdx.y, m = bx >> 1;
        const uint32_t sz = gx - 2u * m < 2u ? gx - 2u * m : 2u;
        if (bx == 2u * m + (by + m) % sz) pipe_run(dc, IC<1>{}, IC<2>{}, IC<1>{}, m);
    };
    if (head_dim == 64) {
        if (pair_coarse) run_pairs(IC<64>{});
        else if (pair2) run_pairs2(IC<64>{});
        else if (vec) run(IC<64>{}, IC<1>{}); else run(IC<64>{}, IC<0>{});
    } else if (D64_ONLY) {
        return;
    } else if (head_dim == 16) {
        if (pair_coarse) run_pairs(IC<16>{});
        else if (pair2) run_pairs2(IC<16>{});
        else if (vec) run(IC<16>{}, IC<1>{}); else run(IC<16>{}, IC<0>{});
    } else if (head_dim == 32) {
        if (pair_coarse) run_pairs(IC<32>{});
        else if (pair2) run_pairs2(IC<32>{});
        else if (vec) run(IC<32>{}, IC<1>{}); else run(IC<32>{}, IC<0>{});
    }
}

}  // namespace

// Each instantiation defines NAME (f16) and NAME_bf16.
#define NC_FLASH_KERNEL(NAME, D, NQ, NS, CAUSAL, VEC)                                          \
    extern "C" __global__ __launch_bounds__(NQ * NS * 64) void NAME(nc_flash_kernel_args a) {        \
        flash_fwd_body<D, NQ, NS, CAUSAL, VEC, false>(a);                                      \
    }                                                                                          \
    extern "C" __global__ __launch_bounds__(NQ * NS * 64) void NAME##_bf16(nc_flash_kernel_args a) { \
        flash_fwd_body<D, NQ, NS, CAUSAL, VEC, true>(a);                                       \
    }

// Generic variants (64-bit addressing, register staging): 16-byte aligned rows whose slices are
// too large for the pipelined kernels' 32-bit buffer offsets.
NC_FLASH_KERNEL(nc_flash_fwd_d16_m64_full, 16, 2, 2, false, true)
NC_FLASH_KERNEL(nc_flash_fwd_d16_m64_causal, 16, 2, 2, true, true)
NC_FLASH_KERNEL(nc_flash_fwd_d32_m64_full, 32, 2, 2, false, true)
NC_FLASH_KERNEL(nc_flash_fwd_d32_m64_causal, 32, 2, 2, true, true)
NC_FLASH_KERNEL(nc_flash_fwd_d64_m64_full, 64, 2, 2, false, true)
NC_FLASH_KERNEL(nc_flash_fwd_d64_m64_causal, 64, 2, 2, true, true)

// The same body in two more geometries: 32 query rows over 8 key-split waves (small grids: 2-3.5x
// the 64-row kernels there) and, at d = 64, 128 rows over 2 key splits (large grids: 1.1-1.4x).
NC_FLASH_KERNEL(nc_flash_fwd_d16_m64_q1s8_full, 16, 1, 8, false, true)
NC_FLASH_KERNEL(nc_flash_fwd_d16_m64_q1s8_causal, 16, 1, 8, true, true)
NC_FLASH_KERNEL(nc_flash_fwd_d32_m64_q1s8_full, 32, 1, 8, false, true)
NC_FLASH_KERNEL(nc_flash_fwd_d32_m64_q1s8_causal, 32, 1, 8, true, true)
NC_FLASH_KERNEL(nc_flash_fwd_d64_m64_q1s8_full, 64, 1, 8, false, true)
NC_FLASH_KERNEL(nc_flash_fwd_d64_m64_q1s8_causal, 64, 1, 8, true, true)
NC_FLASH_KERNEL(nc_flash_fwd_d64_m64_q4s2_full, 64, 4, 2, false, true)
NC_FLASH_KERNEL(nc_flash_fwd_d64_m64_q4s2_causal, 64, 4, 2, true, true)

// Element-wise variants for slices whose base or strides break 16-byte alignment.
NC_FLASH_KERNEL(nc_flash_fwd_d16_m64_full_unaligned, 16, 2, 2, false, false)
NC_FLASH_KERNEL(nc_flash_fwd_d16_m64_causal_unaligned, 16, 2, 2, true, false)
NC_FLASH_KERNEL(nc_flash_fwd_d32_m64_full_unaligned, 32, 2, 2, false, false)
NC_FLASH_KERNEL(nc_flash_fwd_d32_m64_causal_unaligned, 32, 2, 2, true, false)
NC_FLASH_KERNEL(nc_flash_fwd_d64_m64_full_unaligned, 64, 2, 2, false, false)
NC_FLASH_KERNEL(nc_flash_fwd_d64_m64_causal_unaligned, 64, 2, 2, true, false)
NC_FLASH_KERNEL(nc_flash_fwd_d16_m64_q1s8_full_unaligned, 16, 1, 8, false, false)
NC_FLASH_KERNEL(nc_flash_fwd_d16_m64_q1s8_causal_unaligned, 16, 1, 8, true, false)
NC_FLASH_KERNEL(nc_flash_fwd_d32_m64_q1s8_full_unaligned, 32, 1, 8, false, false)
NC_FLASH_KERNEL(nc_flash_fwd_d32_m64_q1s8_causal_unaligned, 32, 1, 8, true, false)
NC_FLASH_KERNEL(nc_flash_fwd_d64_m64_q1s8_full_unaligned, 64, 1, 8, false, false)
NC_FLASH_KERNEL(nc_flash_fwd_d64_m64_q1s8_causal_unaligned, 64, 1, 8, true, false)
NC_FLASH_KERNEL(nc_flash_fwd_d64_m64_q4s2_full_unaligned, 64, 4, 2, false, false)
NC_FLASH_KERNEL(nc_flash_fwd_d64_m64_q4s2_causal_unaligned, 64, 4, 2, true, false)

// Plain 16-byte copy, used only to calibrate rocprofv3 FETCH_SIZE / WRITE_SIZE against a known byte
// count (bench.py --calibrate-copy).
extern "C" __global__ __launch_bounds__(256) void nc_util_copy_b128(const u32x4 *src, u32x4 *dst, uint64_t n16) {
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * 256ull) dst[i] = src[i];
}

// Empty kernel with the flash kernels' argument block: launched with a flash kernel's grid, it
// times the fixed per-launch dispatch and completion cost that no kernel body can remove.
extern "C" __global__ __launch_bounds__(1024) void nc_util_empty(nc_flash_kernel_args a) { (void)a; }

// MFMA ceiling: back-to-back f16 32x32x16 MFMAs on four independent accumulators per wave, with
// operands read once from `ops` (n8 half8 elements). Launched with one 768-thread workgroup per CU:
// 3 waves per SIMD ran this stream fastest (4 waves per SIMD ran it 10-17 % slower), and a second
// workgroup does not fit beside it, so every CU holds the same work. Under full load the chip's clock falls with
// the power that the operands' toggling bits draw, so with operands drawn like a workload's inputs
// this measures the matrix-core rate the chip sustains on such data. out[t] = the sum of thread t's
// accumulators: 2048 * iters when every operand is 1.0.
extern "C" __global__ __launch_bounds__(768) void nc_util_mfma_ceiling(const half8 *ops, uint32_t n8, float *out,
                                                                      uint32_t iters) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    half8 a[4], b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        a[j] = ops[(8u * t + j) % n8];
        b[j] = ops[(8u * t + 4u + j) % n8];
    }
    floatx16 c[4] = {};
    for (uint32_t it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 4; ++j) c[j] = mfma32<false>(a[j], b[j], c[j]);
#pragma unroll
        for (int j = 0; j < 4; ++j) c[j] = mfma32<false>(a[(j + 1) & 3], b[(j + 1) & 3], c[j]);
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) s += c[j][e];
    out[t] = s;
}

// Each instantiation defines NAME (f16) and NAME_bf16.
#define NC_FLASH_PIPE_KERNEL(NAME, D, NQ, NS, CAUSAL, NSTAGE, SUB)                              \
    extern "C" __global__ __launch_bounds__(NQ * NS * 64) void NAME(nc_flash_kernel_args a) {        \
        flash_fwd_pipe_kernel<D, NQ, NS, CAUSAL, NSTAGE, SUB, false>(a);                         \
    }                                                                                          \
    extern "C" __global__ __launch_bounds__(NQ * NS * 64) void NAME##_bf16(nc_flash_kernel_args a) { \
        flash_fwd_pipe_kernel<D, NQ, NS, CAUSAL, NSTAGE, SUB, true>(a);                          \
    }
// With a register budget held to WPE waves per SIMD (512 / WPE VGPRs per wave): two 8-wave
// workgroups of the 70 KB-LDS variants share a CU only if each wave fits in 128 VGPRs.
#define NC_FLASH_PIPE_KERNEL_WPE(NAME, D, NQ, NS, CAUSAL, NSTAGE, SUB, WPE)                             \
    extern "C" __global__ __launch_bounds__(NQ * NS * 64) __attribute__((amdgpu_waves_per_eu(WPE)))     \
    void NAME(nc_flash_kernel_args a) {                                                                 \
        flash_fwd_pipe_kernel<D, NQ, NS, CAUSAL, NSTAGE, SUB, false>(a);                                  \
    }                                                                                                   \
    extern "C" __global__ __launch_bounds__(NQ * NS * 64) __attribute__((amdgpu_waves_per_eu(WPE)))     \
    void NAME##_bf16(nc_flash_kernel_args a) {                                                          \
        flash_fwd_pipe_kernel<D, NQ, NS, CAUSAL, NSTAGE, SUB, true>(a);                                   \
    }

// Pipelined variants: q = query waves (32 rows each), s = key-split waves, p = LDS ring depth.
NC_FLASH_PIPE_KERNEL_WPE(nc_flash_fwd_d64_q8s1p2t2_full, 64, 8, 1, false, 2, 2, 4)
NC_FLASH_PIPE_KERNEL_WPE(nc_flash_fwd_d64_q8s1p2t2_causal, 64, 8, 1, true, 2, 2, 4)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d64_q4s1p2t2_full, 64, 4, 1, false, 2, 2)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d64_q4s1p2t2_causal, 64, 4, 1, true, 2, 2)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d64_q2s4p2_full, 64, 2, 4, false, 2, 1)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d64_q2s4p2_causal, 64, 2, 4, true, 2, 1)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d64_q1s8p2_full, 64, 1, 8, false, 2, 1)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d64_q1s8p2_causal, 64, 1, 8, true, 2, 1)
// Pair split (x): causal query blocks p and nqb-1-p shared by two workgroups that exchange partials.
#define NC_FLASH_XS_KERNEL(NAME, D)                                                                     \
    extern "C" __global__ __launch_bounds__(512) void NAME(nc_flash_kernel_args a) {                     \
        flash_fwd_pipe_kernel<D, 1, 8, true, 2, 1, false, true>(a);                                       \
    }                                                                                                   \
    extern "C" __global__ __launch_bounds__(512) void NAME##_bf16(nc_flash_kernel_args a) {              \
        flash_fwd_pipe_kernel<D, 1, 8, true, 2, 1, true, true>(a);                                        \
    }
NC_FLASH_XS_KERNEL(nc_flash_fwd_d64_q1s8p2x_causal, 64)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d32_q4s1p3_full, 32, 4, 1, false, 3, 1)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d32_q4s1p3_causal, 32, 4, 1, true, 3, 1)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d32_q2s4p2_full, 32, 2, 4, false, 2, 1)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d32_q2s4p2_causal, 32, 2, 4, true, 2, 1)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d32_q1s8p2_full, 32, 1, 8, false, 2, 1)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d32_q1s8p2_causal, 32, 1, 8, true, 2, 1)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d16_q4s1p2t2_full, 16, 4, 1, false, 2, 2)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d16_q4s1p2t2_causal, 16, 4, 1, true, 2, 2)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d16_q2s4p2_full, 16, 2, 4, false, 2, 1)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d16_q2s4p2_causal, 16, 2, 4, true, 2, 1)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d16_q1s8p2_full, 16, 1, 8, false, 2, 1)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d16_q1s8p2_causal, 16, 1, 8, true, 2, 1)
// Private staging with one ring stage, for short sequences (at most three 32-key tiles per wave).
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d64_q1s8p1_full, 64, 1, 8, false, 1, 1)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d64_q1s8p1_causal, 64, 1, 8, true, 1, 1)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d32_q1s8p1_full, 32, 1, 8, false, 1, 1)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d32_q1s8p1_causal, 32, 1, 8, true, 1, 1)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d16_q1s8p1_full, 16, 1, 8, false, 1, 1)
NC_FLASH_PIPE_KERNEL(nc_flash_fwd_d16_q1s8p1_causal, 16, 1, 8, true, 1, 1)

// Dense-layout private-staging kernels: nc_flash_kernel_args as one parameter per field (the first
// seven preloaded into SGPRs; the Makefile builds this code object with
// -amdgpu-kernarg-preload-count=7).
#define NC_KARG_PARAMS                                                                                     \
    const uint16_t *q, const uint16_t *k, const uint16_t *v, float *o, uint64_t seq_len, uint64_t head_dim,  \
        uint64_t q_stride, uint64_t k_stride, uint64_t v_stride, uint64_t o_stride, float scale, uint32_t causal, \
        uint64_t q_row_stride, uint64_t k_row_stride, uint64_t v_row_stride, uint64_t o_row_stride,           \
        uint32_t batch_heads, uint32_t num_q_blocks, void *scratch, uint32_t balance_tail
#define NC_FLASH_DENSE_KERNEL(NAME, D, CAUSAL, NSTAGE)                                                       \
    extern "C" __global__ __launch_bounds__(512) void NAME(NC_KARG_PARAMS) {                                 \
        flash_fwd_dense_kernel<D, 8, CAUSAL, NSTAGE, false>(q, k, v, o, seq_len, head_dim, scale, scratch);   \
    }                                                                                                       \
    extern "C" __global__ __launch_bounds__(512) void NAME##_bf16(NC_KARG_PARAMS) {                          \
        flash_fwd_dense_kernel<D, 8, CAUSAL, NSTAGE, true>(q, k, v, o, seq_len, head_dim, scale, scratch);    \
    }
NC_FLASH_DENSE_KERNEL(nc_flash_fwd_d64_q1s8p2d_causal, 64, true, 2)
NC_FLASH_DENSE_KERNEL(nc_flash_fwd_d64_q1s8p2d_full, 64, false, 2)
NC_FLASH_DENSE_KERNEL(nc_flash_fwd_d64_q1s8p1d_causal, 64, true, 1)
NC_FLASH_DENSE_KERNEL(nc_flash_fwd_d64_q1s8p1d_full, 64, false, 1)
NC_FLASH_DENSE_KERNEL(nc_flash_fwd_d32_q1s8p2d_causal, 32, true, 2)
NC_FLASH_DENSE_KERNEL(nc_flash_fwd_d32_q1s8p2d_full, 32, false, 2)
NC_FLASH_DENSE_KERNEL(nc_flash_fwd_d32_q1s8p1d_causal, 32, true, 1)
NC_FLASH_DENSE_KERNEL(nc_flash_fwd_d32_q1s8p1d_full, 32, false, 1)
NC_FLASH_DENSE_KERNEL(nc_flash_fwd_d16_q1s8p2d_causal, 16, true, 2)
NC_FLASH_DENSE_KERNEL(nc_flash_fwd_d16_q1s8p2d_full, 16, false, 2)
NC_FLASH_DENSE_KERNEL(nc_flash_fwd_d16_q1s8p1d_causal, 16, true, 1)
NC_FLASH_DENSE_KERNEL(nc_flash_fwd_d16_q1s8p1d_full, 16, false, 1)

// Reference-ABI symbols (src/flash_v2.zig:23, src/flash_opt.zig:17, src/flash_h64.zig:21,
// src/flash_h64_bn32.zig:26, src/flash_h64_causal.zig:20, src/kernels.zig:380): one body, launched
// with the reference's grid (ceil(S/16), batch_heads) and 64 or 128 threads; each symbol keeps its
// reference kernel's head_dim domain and causal handling (flash_fwd_refabi's two switches).
// WAVES: staging regions of the symbol's LDS, 4 for the symbols the reference launches with 128
// threads and 2 for those it launches with 64 (src/flash.zig:84-95); a launch may use at most
// WAVES waves.
#define NC_FLASH_REFABI_KERNEL(NAME, ALWAYS_CAUSAL, D64_ONLY, WAVES)                                  \
    extern "C" __global__ __launch_bounds__(256) void NAME(                                           \
        const uint16_t *q, const uint16_t *k, const uint16_t *v, float *o, uint64_t seq_len,          \
        uint64_t head_dim, uint64_t q_stride, uint64_t k_stride, uint64_t v_stride, uint64_t o_stride, \
        float scale, uint32_t causal) {                                                               \
        flash_fwd_refabi<ALWAYS_CAUSAL, D64_ONLY, WAVES>(q, k, v, o, seq_len, head_dim, q_stride, k_stride, \
                                                         v_stride, o_stride, scale, causal);         \
    }
NC_FLASH_REFABI_KERNEL(flash_attention_fwd_v2, false, false, 4)
NC_FLASH_REFABI_KERNEL(flash_attention_fwd_opt, false, false, 2)
NC_FLASH_REFABI_KERNEL(flash_attention_fwd_h64, false, true, 2)
NC_FLASH_REFABI_KERNEL(flash_attention_fwd_h64_bn32, false, true, 4)
NC_FLASH_REFABI_KERNEL(flash_attention_fwd_h64_causal, true, true, 2)
NC_FLASH_REFABI_KERNEL(flash_attention_fwd, false, false, 2)
