// flash.cpp — flash-attention host API (the role of src/flash.zig in the reference).
//
//   nc_flash_options_init / nc_flash_validate   <- flash.Options + validate   (src/flash.zig:5-29)
//   nc_flash_select_kernel[_for]                 <- KernelSelection + selectKernel (src/flash.zig:72-96)
//   nc_flash_launch[_async]                      <- launch + requireLen       (src/flash.zig:31-70, 98-100)
//
// Validation keeps the reference's rules and error (InvalidValue); the optional row strides extend
// them so that a padded row pitch can be described (a layout the reference API cannot express).
// Dispatch keeps the reference's output contract (a kernel name, a label and a thread count) and
// adds the launch geometry, because the gfx950 kernels tile queries in 32/64/128-row blocks rather
// than the fixed 16 of src/config.zig:19 that the reference's callers hard-code.

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdint>
#include <cstring>
#include <limits>

#include "notcute_flash.h"

// hip_api.cpp: the module's workspace for by-name callers, grown (and zeroed) on demand; error text.
extern "C" int nc_internal_module_workspace(nc_module module, size_t bytes, void **out);
extern "C" int nc_internal_fail(int status, const char *what);
// noalloc.hip: the current device's static scratch of the pair-split kernels, and its size.
extern "C" int nc_internal_static_scratch(void **out, size_t *cap);

namespace {

// Kernel families of flash_fwd.hip. Geometry and LDS sizes must agree with Cfg<> / PipeCfg<>.
enum class Family { kPipe, kGeneric };

struct Variant {
    const char *name;
    uint32_t d;
    uint32_t nq;      // query waves (32 rows each)
    uint32_t ns;      // key-split waves
    uint32_t nstage;  // LDS ring depth (pipelined family)
    uint32_t sub;     // 32-key sub-tiles per wave per block (pipelined family)
    bool causal;
    bool aligned;
    Family family;
    bool bf16;  // the `_bf16` twin of the kernel (bf16 Q/K/V)
    bool xsplit = false;  // causal query blocks p and nqb-1-p shared by two workgroups (`x` kernels)
    bool dense = false;   // dense-layout twin of a private-staging kernel (`d` kernels)

    uint32_t bm() const { return 32 * nq; }
    uint32_t bn() const { return 32 * ns * sub; }
    uint32_t threads() const { return 64 * nq * ns; }
    uint32_t lds_bytes() const {
        const uint32_t nw = nq * ns;
        const uint32_t o_bytes = nw * 32 * (d + 4) * 4;
        if (family == Family::kPipe) {
            const uint32_t ring = nstage * 2 * bn() * d * 2;
            // + (m, l) area, + the workgroup's Q tile when key-split waves share it
            // (+ a second Q tile and two exchange words for the pair-split kernels)
            return (ring > o_bytes ? ring : o_bytes) + nw * 32 * 2 * 4 + (ns > 1 ? bm() * d * 2 : 0) +
                   (xsplit ? bm() * d * 2 + 16 : 0);
        }
        const uint32_t dv = d < 32 ? 32 : d;
        const uint32_t stage = bn() * (d + 8) * 2 + dv * (bn() + 8) * 2;
        return (stage > o_bytes ? stage : o_bytes) + nw * 32 * 2 * 4;
    }
};

#define PIPE(D, NQ, NS, P, C, T, BF) {"nc_flash_fwd_d" #D "_q" #NQ "s" #NS "p" #P "_" C T, D, NQ, NS, P, 1, \
                                      C[0] == 'c', true, Family::kPipe, BF}
// Pair split (flash_fwd.hip's XS kernels): d=64 causal, one query wave, eight key splits.
#define PIPEX(D, T, BF) {"nc_flash_fwd_d" #D "_q1s8p2x_causal" T, D, 1, 8, 2, 1, true, true, Family::kPipe, BF, true}
// Dense-layout private-staging kernels (flash_fwd.hip's `d` kernels: one parameter per field of the
// argument block, slot from a 3-D workgroup id).
#define PIPED(D, P, C, T, BF) {"nc_flash_fwd_d" #D "_q1s8p" #P "d_" C T, D, 1, 8, P, 1, C[0] == 'c', true, \
                               Family::kPipe, BF, false, true}
#define PIPED4(D, T, BF) PIPED(D, 2, "causal", T, BF), PIPED(D, 2, "full", T, BF), PIPED(D, 1, "causal", T, BF), \
    PIPED(D, 1, "full", T, BF)
// Two 32-key sub-tiles per wave per block ("t2": 32*NS*2 keys per block).
#define PIPE2(D, NQ, NS, P, C, T, BF) {"nc_flash_fwd_d" #D "_q" #NQ "s" #NS "p" #P "t2_" C T, D, NQ, NS, P, 2, \
                                       C[0] == 'c', true, Family::kPipe, BF}
#define GEN(D, C, A, SUF, T, BF) {"nc_flash_fwd_d" #D "_m64_" C SUF T, D, 2, 2, 1, 1, C[0] == 'c', A, \
                                  Family::kGeneric, BF}
// The generic body in other geometries (32 rows x 8 key splits; 128 rows x 2 key splits).
#define GENG(D, NQ, NS, C, A, SUF, T, BF) {"nc_flash_fwd_d" #D "_m64_q" #NQ "s" #NS "_" C SUF T, D, NQ, NS, 1, 1, \
                                           C[0] == 'c', A, Family::kGeneric, BF}
#define GENG2(D, NQ, NS, T, BF) GENG(D, NQ, NS, "full", true, "", T, BF), GENG(D, NQ, NS, "causal", true, "", T, BF), \
    GENG(D, NQ, NS, "full", false, "_unaligned", T, BF), GENG(D, NQ, NS, "causal", false, "_unaligned", T, BF)
// Every kernel of the family, once per element type (T: name suffix, BF: bf16).
#define VARIANTS(T, BF)                                                                                         \
    PIPE2(64, 8, 1, 2, "full", T, BF), PIPE2(64, 8, 1, 2, "causal", T, BF), PIPE2(64, 4, 1, 2, "full", T, BF),  \
    PIPE2(64, 4, 1, 2, "causal", T, BF), PIPE(64, 2, 4, 2, "full", T, BF), PIPE(64, 2, 4, 2, "causal", T, BF),  \
    PIPE(64, 1, 8, 2, "full", T, BF), PIPE(64, 1, 8, 2, "causal", T, BF), PIPE(32, 4, 1, 3, "full", T, BF),     \
    PIPE(32, 4, 1, 3, "causal", T, BF), PIPE(32, 2, 4, 2, "full", T, BF), PIPE(32, 2, 4, 2, "causal", T, BF),   \
    PIPE(32, 1, 8, 2, "full", T, BF), PIPE(32, 1, 8, 2, "causal", T, BF), PIPE2(16, 4, 1, 2, "full", T, BF),    \
    PIPE2(16, 4, 1, 2, "causal", T, BF), PIPE(16, 2, 4, 2, "full", T, BF), PIPE(16, 2, 4, 2, "causal", T, BF),  \
    PIPE(16, 1, 8, 2, "full", T, BF), PIPE(16, 1, 8, 2, "causal", T, BF),                                      \
    GEN(16, "full", true, "", T, BF), GEN(16, "causal", true, "", T, BF), GEN(32, "full", true, "", T, BF),     \
    GEN(32, "causal", true, "", T, BF), GEN(64, "full", true, "", T, BF), GEN(64, "causal", true, "", T, BF),   \
    GEN(16, "full", false, "_unaligned", T, BF), GEN(16, "causal", false, "_unaligned", T, BF),                \
    GEN(32, "full", false, "_unaligned", T, BF), GEN(32, "causal", false, "_unaligned", T, BF),                \
    GEN(64, "full", false, "_unaligned", T, BF), GEN(64, "causal", false, "_unaligned", T, BF), PIPEX(64, T, BF), \
    GENG2(16, 1, 8, T, BF), GENG2(32, 1, 8, T, BF), GENG2(64, 1, 8, T, BF), GENG2(64, 4, 2, T, BF),          \
    PIPE(64, 1, 8, 1, "full", T, BF), PIPE(64, 1, 8, 1, "causal", T, BF), PIPE(32, 1, 8, 1, "full", T, BF),   \
    PIPE(32, 1, 8, 1, "causal", T, BF), PIPE(16, 1, 8, 1, "full", T, BF), PIPE(16, 1, 8, 1, "causal", T, BF), \
    PIPED4(64, T, BF), PIPED4(32, T, BF), PIPED4(16, T, BF)

const Variant kVariants[] = {VARIANTS("", false), VARIANTS("_bf16", true)};
#undef VARIANTS
#undef PIPE
#undef PIPE2
#undef PIPEX
#undef PIPED
#undef PIPED4
#undef GEN
#undef GENG
#undef GENG2

const Variant *find_pipe(uint32_t d, uint32_t nq, uint32_t ns, bool causal, bool bf16) {
    for (const auto &v : kVariants)
        if (v.family == Family::kPipe && v.d == d && v.nq == nq && v.ns == ns && v.causal == causal && v.bf16 == bf16 &&
            !v.xsplit && !v.dense)
            return &v;
    return nullptr;
}

// The same, with a given ring depth (find_pipe returns the first in the table: the two-stage one).
const Variant *find_pipe_stages(uint32_t d, uint32_t nq, uint32_t ns, uint32_t nstage, bool causal, bool bf16) {
    for (const auto &v : kVariants)
        if (v.family == Family::kPipe && v.d == d && v.nq == nq && v.ns == ns && v.nstage == nstage &&
            v.causal == causal && v.bf16 == bf16 && !v.xsplit && !v.dense)
            return &v;
    return nullptr;
}

// The dense-layout twin of a private-staging kernel, if there is one.
const Variant *find_dense(const Variant &base) {
    for (const auto &v : kVariants)
        if (v.dense && v.d == base.d && v.nq == base.nq && v.ns == base.ns && v.nstage == base.nstage &&
            v.causal == base.causal && v.bf16 == base.bf16)
            return &v;
    return nullptr;
}

// The table entry of a kernel name (a selection's name points into the table), or null.
const Variant *variant_of(const char *name) {
    if (!name) return nullptr;
    for (const auto &v : kVariants)
        if (v.name == name) return &v;
    for (const auto &v : kVariants)
        if (std::strcmp(v.name, name) == 0) return &v;
    return nullptr;
}

const Variant *find_xsplit(uint32_t d, bool bf16) {
    for (const auto &v : kVariants)
        if (v.xsplit && v.d == d && v.bf16 == bf16) return &v;
    return nullptr;
}

// Pairs of workgroups of a pair-split launch, and its scratch: the fixed counter region, then two
// slots per pair of 32 x d f32 partial O plus 32 (m, l) pairs (flash_fwd.hip's pair exchange).
uint64_t xsplit_pairs(uint64_t batch_heads, uint64_t seq_len) { return batch_heads * (((seq_len + 31) / 32) / 2); }
uint64_t xsplit_scratch_bytes(uint64_t batch_heads, uint64_t seq_len, uint64_t d) {
    return NC_XS_COUNTER_BYTES + xsplit_pairs(batch_heads, seq_len) * 2 * (32 * d * 4 + 32 * 8);
}

const Variant *find_generic(uint32_t d, uint32_t nq, uint32_t ns, bool causal, bool aligned, bool bf16) {
    for (const auto &v : kVariants)
        if (v.family == Family::kGeneric && v.d == d && v.nq == nq && v.ns == ns && v.causal == causal &&
            v.aligned == aligned && v.bf16 == bf16)
            return &v;
    return nullptr;
}

// Geometry of the generic kernels (rows past 16-byte alignment or past 32-bit offsets), from GPU
// timings of the three on 132 shapes (d 16/32/64, BH 1-128, S 256-8192, causal and not), where
// these picks come within 0.6 % of the per-shape best on average and the 64-row kernel alone
// averaged 1.30-1.83x: 32 rows x 8 key splits while the grid is small, 128 x 2 for large d=64
// grids, the 64-row, 4-wave kernel between.
const Variant *choose_generic(const nc_flash_options &o, bool aligned) {
    const uint32_t d = (uint32_t)o.head_dim;
    const bool causal = o.causal != 0, bf = o.element_type == NC_ELEMENT_BF16;
    const uint64_t S = o.seq_len, w32 = (S + 31) / 32 * o.batch_heads, w128 = (S + 127) / 128 * o.batch_heads;
    bool small;
    if (d == 64) {
        if (w128 >= (causal ? 384u : 256u)) return find_generic(d, 4, 2, causal, aligned, bf);
        small = causal ? (w32 <= 384 || (w32 <= 512 && S >= 1024)) : w32 <= 256;
    } else if (d == 32) {
        small = w32 <= 768 || (w32 <= 1024 && S >= (causal ? 1024u : 4096u));
    } else {
        small = w32 <= 768 || (causal ? (w32 <= 2048 && S >= 1024) : (w32 <= 1024 && S >= 512));
    }
    return small ? find_generic(d, 1, 8, causal, aligned, bf) : find_generic(d, 2, 2, causal, aligned, bf);
}

uint64_t row_stride_of(uint64_t rs, uint64_t d) { return rs == 0 ? d : rs; }

bool mul_overflows(uint64_t a, uint64_t b, uint64_t *out) {
    if (a != 0 && b > std::numeric_limits<uint64_t>::max() / a) return true;
    *out = a * b;
    return false;
}

// The reference's selectKernel, restated (src/flash.zig:78-96), so every selection records which
// reference kernel it stands in for.
const char *reference_kernel(const nc_flash_options &o) {
    if (o.head_dim <= 32 && o.seq_len <= 256 && o.batch_heads <= 8) return "flash_attention_fwd_v2";
    if (o.head_dim == 64 && !o.causal && o.seq_len <= 256 && o.batch_heads <= 8) return "flash_attention_fwd_v2";
    if (o.head_dim == 64 && o.seq_len >= 512) return "flash_attention_fwd_h64_bn32";
    if (o.head_dim == 64) return "flash_attention_fwd_h64";
    return "flash_attention_fwd_opt";
}

// MI355X dispatch (256 CUs): at d = 64 and 32 every pipelined kernel of the head size is priced by a
// cost model and the cheapest is launched (d = 16: fitted thresholds, in choose_pipe). A kernel's
// workgroups are dealt to the CUs in block order (heaviest causal query blocks first), so the
// busiest CU holds workgroups 0, 256, 512, ... . It runs up to
// wg_per_cu of them at once (from each kernel's registers and LDS); each resident workgroup needs
// rho + steps units of work, steps being its busiest wave's sequential 32-key tiles (the padded key
// blocks up to its last visible key), and advances one unit per max(lat, k * waves_per_simd * tau)
// us while k workgroups share the CU: lat is one wave's latency-bound tile, tau a tile's share of a
// SIMD once waves interleave. The estimate is a + that CU's finishing time. Partial query and key
// blocks, causal imbalance and how full the CUs are all enter through the steps and the sharing,
// which fixed grid-size thresholds miss off a power-of-two grid. (a, rho, lat, tau) were fitted per
// kernel to interleaved GPU timings of every variant on 245 (d=64) and 244 (d=32) shapes (BH 1-1024,
// S 64-16384, causal and not; a grid, an off-grid set and a random set). On 100 random shapes per
// head size timed after the fit the picks average 1.003x (d=64) and 1.006x (d=32) the per-shape
// best, where the threshold rules they replace averaged 1.052x and 1.023x; on 50 bf16 shapes each,
// 1.010x and 1.006x (thresholds: 1.046x and 1.049x). The bf16 twins have the same instruction
// stream and use the same model.
// `balance`: the non-causal kernel orders its waves by remaining work in the grid's last
// wg_per_cu * CUs workgroups (nc_flash_kernel_args.balance_tail), where that was measured faster.
struct PipeModel {
    uint32_t d, nq, ns, wg_per_cu, waves_per_simd;
    float a, rho, lat, tau;
    bool balance;
};
const PipeModel kPipeModels[] = {
    {64, 8, 1, 2, 2, 2.3643f, 3.7198f, 0.5110f, 0.2491f, true},    // q8s1p2t2
    {64, 4, 1, 4, 1, 1.9664f, 4.3401f, 0.4105f, 0.2735f, true},    // q4s1p2t2
    {64, 2, 4, 2, 2, 2.0057f, 2.5877f, 0.5000f, 0.3134f, true},    // q2s4p2
    {64, 1, 8, 1, 2, 0.4023f, 2.9534f, 0.3000f, 0.3978f, false},   // q1s8p2
    {32, 4, 1, 5, 1, 2.0217f, 2.5512f, 0.3837f, 0.1863f, false},   // q4s1p3
    {32, 2, 4, 2, 2, 1.7707f, 2.6393f, 0.5084f, 0.2020f, true},    // q2s4p2
    {32, 1, 8, 2, 2, 1.6322f, 1.5959f, 0.5621f, 0.2483f, false},   // q1s8p2
};

// CUs of the current device, read once per device (0 without one).
uint32_t device_cu_count() {
    constexpr int kMaxDevices = 64;
    static std::atomic<uint32_t> cus[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
    uint32_t n = cus[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        int c = 0;
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) return 0;
        n = (uint32_t)c;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// nc_flash_kernel_args.balance_tail for a selection: the last wg_per_cu * CUs workgroups of a
// non-causal grid on a kernel marked `balance`, once the grid holds more workgroups than the device
// has CUs (with one workgroup per CU there is nothing to balance, and the priority changes were
// measured to cost up to 4 % there); else 0.
uint32_t balance_tail_for(const nc_flash_options &o, const nc_flash_kernel_selection &sel) {
    if (o.causal || !sel.name) return 0;
    const Variant *v = nullptr;
    for (const auto &x : kVariants)
        if (x.name == sel.name) {  // a selection's name points into the table
            v = &x;
            break;
        }
    if (!v || v->family != Family::kPipe || v->nq == 1) return 0;
    const PipeModel *m = nullptr;
    for (const auto &pm : kPipeModels)
        if (pm.d == v->d && pm.nq == v->nq && pm.ns == v->ns) m = &pm;
    if (!m || !m->balance) return 0;
    const uint64_t grid = (uint64_t)sel.grid[0] * sel.grid[1] * sel.grid[2];
    const uint32_t cus = device_cu_count();
    if (cus == 0 || grid <= cus) return 0;
    return (uint32_t)std::min<uint64_t>(grid, (uint64_t)cus * m->wg_per_cu);
}

// Sequential 32-key tiles of the busiest wave of query block qb.
uint64_t pipe_steps(const Variant &v, uint64_t S, bool causal, uint64_t qb) {
    const uint64_t kv = causal ? std::min<uint64_t>(S, (qb + 1) * v.bm()) : S;
    if (v.nq == 1) return ((kv + 31) / 32 + v.ns - 1) / v.ns;  // private staging: wave s takes tiles s + ns*i
    return (kv + v.bn() - 1) / v.bn() * v.sub;
}

double pipe_cost(const PipeModel &m, const Variant &v, uint64_t batch_heads, uint64_t S, bool causal) {
    const uint64_t nqb = (S + v.bm() - 1) / v.bm(), n = nqb * batch_heads, ncu = (n + 255) / 256;
    auto per = [&](uint64_t k) { return std::max<double>(m.lat, (double)k * m.waves_per_simd * m.tau); };
    if (!causal) {  // equal workgroups: rounds of wg_per_cu, then the remainder
        const double job = (double)pipe_steps(v, S, false, 0) + m.rho;
        const uint64_t full = ncu / m.wg_per_cu, rem = ncu % m.wg_per_cu;
        return m.a + job * ((double)full * per(m.wg_per_cu) + (rem ? per(rem) : 0.0));
    }
    auto job = [&](uint64_t i) { return (double)pipe_steps(v, S, true, nqb - 1 - (256 * i) / batch_heads) + m.rho; };
    double t = 0.0;
    if (ncu > 512) {  // the CU stays full but for a short tail: its 1/256 share of all the work
        // (over at most 4096 query blocks, evenly strided: steps grow linearly with the block)
        const uint64_t stride = nqb > 4096 ? (nqb + 4095) / 4096 : 1;
        uint64_t counted = 0;
        for (uint64_t qb = 0; qb < nqb; qb += stride, ++counted) t += (double)pipe_steps(v, S, true, qb);
        t = t * (double)nqb / (double)counted * (double)batch_heads / 256.0 + (double)ncu * m.rho;
        return m.a + t * per(m.wg_per_cu) / m.wg_per_cu;
    }
    double act[8];
    uint32_t na = 0;
    uint64_t i = 0;
    for (;;) {
        while (na < m.wg_per_cu && i < ncu) act[na++] = job(i++);
        if (na == 0) break;
        double mn = act[0];
        for (uint32_t r = 1; r < na; ++r) mn = std::min(mn, act[r]);
        t += mn * per(na);
        uint32_t k = 0;
        for (uint32_t r = 0; r < na; ++r)
            if (act[r] - mn > 1e-9) act[k++] = act[r] - mn;
        na = k;
    }
    return m.a + t;
}

const Variant *choose_pipe_layout(const nc_flash_options &o);

// Private staging (one query wave) with one ring stage on short sequences: with at most three
// 32-key tiles per wave, the second stage's prologue costs more than it hides. Measured against the
// two-stage kernels on 58 shapes (d 16/32/64, BH 1-32, S 32-2048): 2-10 % faster up to S = 768 (d=64
// non-causal: 512), 1-6 % slower from S = 1024 on those grids of at most 256 workgroups.
const Variant *choose_pipe(const nc_flash_options &o) {
    const Variant *v = choose_pipe_layout(o);
    const bool causal = o.causal != 0;
    // At d = 64 it is also faster wherever a CU runs several of the workgroups, up to 4096 of them
    // (S > 768, mean of p1/p2 over 311 shapes: causal 513-4096 workgroups 0.89-0.92x, worst 1.04x;
    // non-causal 257-4096 0.91-0.96x, worst 1.03x). It is slower in one round (up to 256: 1.04x)
    // and on large causal grids (over 4096: up to 1.63x); at d = 32 and 16 the two are within 2 %.
    const uint64_t wg32 = (o.seq_len + 31) / 32 * o.batch_heads;
    const bool shared_cu = wg32 >= (causal ? 513u : 257u) && wg32 <= 4096u;
    const bool short_seq = o.seq_len <= (v && v->d == 64 && !causal ? 512u : 768u);
    if (v && v->nq == 1 && (short_seq || (v->d == 64 && shared_cu))) {
        const Variant *p1 = find_pipe_stages(v->d, 1, v->ns, 1, causal, v->bf16);
        if (p1) v = p1;
    }
    return v;
}

const Variant *choose_pipe_layout(const nc_flash_options &o) {
    const uint32_t d = (uint32_t)o.head_dim;
    const bool causal = o.causal != 0;
    const bool bf = o.element_type == NC_ELEMENT_BF16;
    if (d == 16) {
        // d = 16 tiles are cheap next to their softmax and staging, and the model above picks worse
        // there (1.010x the per-shape best in cross-validation) than these fitted thresholds
        // (1.008-1.011x on two random sets timed after their fit, f16 and bf16): q4s1 from 384-1536 of
        // its workgroups, more for longer sequences, then q2s4 from 192-768 of its own.
        const uint64_t S = o.seq_len, bh = o.batch_heads;
        const uint64_t w128 = (S + 127) / 128 * bh, w64 = (S + 63) / 64 * bh;
        const uint64_t need4 = S <= 512 ? 384u : S <= (causal ? 2048u : 1024u) ? 768u : 1536u;
        const uint64_t need2 = S <= (causal ? 512u : 256u) ? 192u : S <= 1024 ? 384u : 768u;
        if (w128 >= need4) return find_pipe(d, 4, 1, causal, bf);
        if (w64 >= need2) return find_pipe(d, 2, 4, causal, bf);
        return find_pipe(d, 1, 8, causal, bf);
    }
    const Variant *best = nullptr, *q1 = nullptr;
    double best_t = 0.0, q1_t = 0.0;
    for (const auto &m : kPipeModels) {
        if (m.d != d) continue;
        const Variant *v = find_pipe(d, m.nq, m.ns, causal, bf);
        if (!v) continue;
        const double t = pipe_cost(m, *v, o.batch_heads, o.seq_len, causal);
        if (m.nq == 1) {
            q1 = v;
            q1_t = t;
        }
        if (!best || t < best_t) {
            best = v;
            best_t = t;
        }
    }
    // The q1s8 row fits worst (0.24 rms-log) and over-prices few-head causal d = 64 shapes, where
    // q1s8 beat the picked q2s4 by up to 1.27x (BH=6 S=2048: 10.9 against 13.9 us). Within 10 % of
    // q2s4's estimate, q1s8 is taken: 1.021x -> 1.014x the per-shape best on 70 random shapes,
    // 1.022x -> 1.012x on 56 few-head ones, no worse on the four 345-shape sets of the fit; on 56
    // random causal shapes timed afterwards (BH 1-64, S 1024-16384), 1.039x -> 1.017x.
    if (d == 64 && causal && best && best->nq == 2 && q1 && q1_t <= 1.1 * best_t) return q1;
    return best;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Every tensor a stack of packed slices: slice stride seq_len * d elements, row stride d.
bool dense_layout(const nc_flash_options &o) {
    const uint64_t d = o.head_dim, slice = o.seq_len * d;
    return row_stride_of(o.q_row_stride, d) == d && row_stride_of(o.k_row_stride, d) == d &&
           row_stride_of(o.v_row_stride, d) == d && row_stride_of(o.o_row_stride, d) == d && o.q_stride == slice &&
           o.k_stride == slice && o.v_stride == slice && o.o_stride == slice;
}

int select_impl(const nc_flash_options *opts, bool vec_ok, nc_flash_kernel_selection *out) {
    if (!out) return NC_ERROR_INVALID_VALUE;
    int st = nc_flash_validate(opts);
    if (st) return st;
    const nc_flash_options &o = *opts;
    const uint64_t d = o.head_dim;
    const uint64_t rows[4] = {row_stride_of(o.q_row_stride, d), row_stride_of(o.k_row_stride, d),
                              row_stride_of(o.v_row_stride, d), row_stride_of(o.o_row_stride, d)};
    // 16-byte vector path: every Q/K/V row start is 16-byte aligned and O rows are float4 aligned.
    const bool strides_ok = o.q_stride % 8 == 0 && o.k_stride % 8 == 0 && o.v_stride % 8 == 0 &&
                            o.o_stride % 4 == 0 && rows[0] % 8 == 0 && rows[1] % 8 == 0 && rows[2] % 8 == 0 &&
                            rows[3] % 4 == 0;
    const bool aligned = vec_ok && strides_ok;
    // The pipelined kernels address each Q/K/V slice with 32-bit buffer offsets, including up to
    // one block (<= 256 rows) past seq_len.
    uint64_t max_row = rows[0] > rows[1] ? rows[0] : rows[1];
    max_row = max_row > rows[2] ? max_row : rows[2];
    const bool offsets_fit = max_row < (1ull << 30) && (o.seq_len + 512) * max_row * 2 < (1ull << 31);
    const Variant *v = (aligned && offsets_fit)
                           ? choose_pipe(o)
                           : choose_generic(o, aligned);
    if (!v) return NC_ERROR_NOT_FOUND;
    // Long causal sequences over few heads on the private-staging kernel: pair the light and heavy
    // query blocks so that every workgroup takes about half the heaviest block's keys. It pays once
    // the whole grid runs at once (one workgroup per CU) and the heaviest block is long enough to
    // outweigh the ~1.2 us exchange between the two workgroups of a pair: measured on MI355X,
    // BH=1 S=8192 23.4 -> 18.6 us, BH=2 S=4096 13.4 -> 12.3 us, but c3 (32 query blocks) 5.9 -> 7.5 us
    // and grids beyond 256 workgroups slower too.
    const uint64_t nqb32 = (o.seq_len + 31) / 32;
    if (v->family == Family::kPipe && v->causal && v->nq == 1 && v->d == 64 && nqb32 >= 96 &&
        nqb32 * o.batch_heads <= 256 && xsplit_pairs(o.batch_heads, o.seq_len) <= NC_XS_MAX_PAIRS) {
        const Variant *x = find_xsplit(v->d, v->bf16);
        if (x) v = x;
    }
    const uint64_t nqb = (o.seq_len + v->bm() - 1) / v->bm();
    uint64_t grid = 0;
    if (mul_overflows(nqb, o.batch_heads, &grid) || grid > 0xffffffffull) return NC_ERROR_OVERFLOW;
    uint32_t g3[3] = {(uint32_t)grid, 1u, 1u};
    // Packed slices on a private-staging kernel: its dense-layout twin, whose waves reach their first
    // loads without reading the argument block from memory. Measured on MI355X against the same
    // kernel with the argument block (interleaved graph replays, bitwise-identical output): c3 5.71
    // -> 5.49 us, BH=8 S=1536 causal 8.50 -> 8.16 us, BH=8 S=2048 causal 10.80 -> 10.52 us. Grid
    // (8, BH/8, nqb) or (BH, 1, nqb): the same workgroups in the same linear order as the 1-D grid.
    if (v->family == Family::kPipe && v->nq == 1 && !v->xsplit && dense_layout(o) && nqb <= 65535) {
        const Variant *dv = find_dense(*v);
        const uint64_t bh = o.batch_heads;
        if (dv && (bh % 8 == 0 ? bh / 8 <= 65535 : bh <= 0x7fffffffu)) {  // grid y, z <= 65535; x < 2^31
            v = dv;
            if (bh % 8 == 0) {
                g3[0] = 8;
                g3[1] = (uint32_t)(bh / 8);
            } else {
                g3[0] = (uint32_t)bh;
            }
            g3[2] = (uint32_t)nqb;
        }
    }
    // The dispatch packet holds each grid dimension in work-items, as 32 bits.
    if ((uint64_t)g3[0] * v->threads() > 0xffffffffull) return NC_ERROR_OVERFLOW;
    std::memset(out, 0, sizeof *out);
    out->name = v->name;
    out->label = v->name;
    out->reference_name = reference_kernel(o);
    out->threads = v->threads();
    out->grid[0] = g3[0];
    out->grid[1] = g3[1];
    out->grid[2] = g3[2];
    out->block_m = v->bm();
    out->block_n = v->bn();
    out->kv_splits = v->ns;
    out->lds_bytes = v->lds_bytes();
    out->aligned = aligned ? 1u : 0u;
    out->scratch_bytes = v->xsplit ? xsplit_scratch_bytes(o.batch_heads, o.seq_len, d) : 0;
    return NC_SUCCESS;
}

}  // namespace

extern "C" {

void nc_flash_options_init(nc_flash_options *opts) {
    if (!opts) return;
    std::memset(opts, 0, sizeof *opts);
    opts->batch_heads = 1;  // src/flash.zig:6
    opts->causal = 0;       // src/flash.zig:14
}

int nc_flash_validate(const nc_flash_options *opts) {
    if (!opts) return NC_ERROR_INVALID_VALUE;
    const nc_flash_options &o = *opts;
    if (o.batch_heads == 0 || o.seq_len == 0) return NC_ERROR_INVALID_VALUE;                   // :17
    if (o.head_dim != 16 && o.head_dim != 32 && o.head_dim != 64) return NC_ERROR_INVALID_VALUE; // :18
    if (o.element_type != NC_ELEMENT_F16 && o.element_type != NC_ELEMENT_BF16) return NC_ERROR_INVALID_VALUE;
    const uint64_t d = o.head_dim;
    const uint64_t rows[4] = {row_stride_of(o.q_row_stride, d), row_stride_of(o.k_row_stride, d),
                              row_stride_of(o.v_row_stride, d), row_stride_of(o.o_row_stride, d)};
    const uint64_t slices[4] = {o.q_stride, o.k_stride, o.v_stride, o.o_stride};
    for (int i = 0; i < 4; ++i) {
        if (rows[i] < d) return NC_ERROR_INVALID_VALUE;
        // Smallest slice that holds seq_len rows: (S-1)*row + d; with row == d this is the
        // reference's S*d (src/flash.zig:20-27).
        uint64_t span = 0;
        if (mul_overflows(o.seq_len - 1, rows[i], &span) || span > std::numeric_limits<uint64_t>::max() - d)
            return NC_ERROR_OVERFLOW;
        if (slices[i] < span + d) return NC_ERROR_INVALID_VALUE;
        uint64_t total = 0;
        if (mul_overflows(o.batch_heads, slices[i], &total)) return NC_ERROR_OVERFLOW;
    }
    // The kernels index rows and keys with 32-bit integers.
    if (o.seq_len > (uint64_t)std::numeric_limits<int32_t>::max() - 256) return NC_ERROR_INVALID_VALUE;
    if (o.batch_heads > 0xffffffffull) return NC_ERROR_INVALID_VALUE;
    return NC_SUCCESS;
}

int nc_flash_select_kernel(const nc_flash_options *opts, nc_flash_kernel_selection *out) {
    return select_impl(opts, true, out);
}

int nc_flash_select_kernel_for(const nc_flash_options *opts, const void *q, const void *k, const void *v,
                               const void *o, nc_flash_kernel_selection *out) {
    return select_impl(opts, aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o), out);
}

int nc_flash_pack_args(const nc_flash_options *opts, const nc_flash_kernel_selection *sel, const uint16_t *q,
                       const uint16_t *k, const uint16_t *v, float *o, nc_flash_kernel_args *out) {
    if (!opts || !sel || !out || sel->block_m == 0) return NC_ERROR_INVALID_VALUE;
    const nc_flash_options &op = *opts;
    std::memset(out, 0, sizeof *out);
    out->q = q;
    out->k = k;
    out->v = v;
    out->o = o;
    out->seq_len = op.seq_len;
    out->head_dim = op.head_dim;
    out->q_stride = op.q_stride;
    out->k_stride = op.k_stride;
    out->v_stride = op.v_stride;
    out->o_stride = op.o_stride;
    out->scale = op.scale;
    out->causal = op.causal ? 1u : 0u;
    out->q_row_stride = row_stride_of(op.q_row_stride, op.head_dim);
    out->k_row_stride = row_stride_of(op.k_row_stride, op.head_dim);
    out->v_row_stride = row_stride_of(op.v_row_stride, op.head_dim);
    out->o_row_stride = row_stride_of(op.o_row_stride, op.head_dim);
    out->batch_heads = (uint32_t)op.batch_heads;
    out->num_q_blocks = (uint32_t)((op.seq_len + sel->block_m - 1) / sel->block_m);
    out->balance_tail = balance_tail_for(op, *sel);
    return NC_SUCCESS;
}

}  // extern "C"

namespace {

// flash.launch for every entry point: the scratch of a kernel that needs one (the pair-split
// kernels) is the caller's buffer of scratch_cap bytes, or with scratch == nullptr the library's
// static scratch on the current device (set up by nc_init), so a launch allocates nothing and does
// not synchronise (src/flash.zig:31-70).
int flash_launch_impl(nc_module module, const uint16_t *q, size_t q_len, const uint16_t *k, size_t k_len,
                      const uint16_t *v, size_t v_len, float *o, size_t o_len, const nc_flash_options *opts,
                      nc_stream stream, void *scratch, size_t scratch_cap) {
    int st = nc_flash_validate(opts);  // src/flash.zig:39
    if (st) return st;
    if (!module || !q || !k || !v || !o) return NC_ERROR_INVALID_VALUE;
    // requireLen (src/flash.zig:40-43, 98-100): each buffer holds batch_heads full slices.
    const uint64_t need[4] = {opts->batch_heads * opts->q_stride, opts->batch_heads * opts->k_stride,
                              opts->batch_heads * opts->v_stride, opts->batch_heads * opts->o_stride};
    const uint64_t have[4] = {q_len, k_len, v_len, o_len};
    for (int i = 0; i < 4; ++i)
        if (have[i] < need[i]) return NC_ERROR_INVALID_VALUE;

    nc_flash_kernel_selection sel;
    st = nc_flash_select_kernel_for(opts, q, k, v, o, &sel);
    if (st) return st;
    nc_function fn = nullptr;
    st = nc_module_get_function(&fn, module, sel.name);
    if (st) return st;
    nc_flash_kernel_args args;
    st = nc_flash_pack_args(opts, &sel, q, k, v, o, &args);
    if (st) return st;
    if (sel.scratch_bytes) {
        if (!scratch) {
            st = nc_internal_static_scratch(&scratch, &scratch_cap);
            if (st) return st;
        }
        if (sel.scratch_bytes > scratch_cap) {
            char msg[200];
            std::snprintf(msg, sizeof msg, "flash launch: %s needs %llu bytes of scratch, more than the %llu available",
                          sel.name, (unsigned long long)sel.scratch_bytes, (unsigned long long)scratch_cap);
            return nc_internal_fail(NC_ERROR_INVALID_VALUE, msg);
        }
        args.scratch = scratch;
    }
    nc_launch_config cfg;
    std::memset(&cfg, 0, sizeof cfg);
    cfg.grid[0] = sel.grid[0];
    cfg.grid[1] = sel.grid[1];
    cfg.grid[2] = sel.grid[2];
    cfg.block[0] = sel.threads;
    cfg.block[1] = 1;
    cfg.block[2] = 1;
    cfg.shared_mem_bytes = 0;
    cfg.stream = stream;
    void *params[NC_FLASH_MAX_KERNEL_PARAMS];
    uint32_t count = 0;
    st = nc_flash_kernel_params(sel.name, &args, params, NC_FLASH_MAX_KERNEL_PARAMS, &count);
    if (st) return st;
    return nc_function_launch(fn, &cfg, params);
}

}  // namespace

extern "C" {

int nc_flash_launch_async(nc_module module, const uint16_t *q, size_t q_len, const uint16_t *k, size_t k_len,
                          const uint16_t *v, size_t v_len, float *o, size_t o_len, const nc_flash_options *opts,
                          nc_stream stream) {
    return flash_launch_impl(module, q, q_len, k, k_len, v, v_len, o, o_len, opts, stream, nullptr, 0);
}

// For noalloc.hip: the same launch with a caller-provided scratch buffer of `cap` bytes (never the
// module's workspace); NC_ERROR_INVALID_VALUE when the selected kernel needs more than `cap`.
int nc_internal_flash_launch_scratch(nc_module module, const uint16_t *q, size_t q_len, const uint16_t *k,
                                     size_t k_len, const uint16_t *v, size_t v_len, float *o, size_t o_len,
                                     const nc_flash_options *opts, nc_stream stream, void *scratch, size_t cap) {
    if (!scratch) return NC_ERROR_INVALID_VALUE;
    return flash_launch_impl(module, q, q_len, k, k_len, v, v_len, o, o_len, opts, stream, scratch, cap);
}

int nc_flash_launch(nc_module module, const uint16_t *q, size_t q_len, const uint16_t *k, size_t k_len,
                    const uint16_t *v, size_t v_len, float *o, size_t o_len, const nc_flash_options *opts) {
    return nc_flash_launch_async(module, q, q_len, k, k_len, v, v_len, o, o_len, opts, nullptr);
}

int nc_flash_kernel_params(const char *name, nc_flash_kernel_args *args, void **params, uint32_t capacity,
                           uint32_t *count) {
    if (!name || !args || !params || !count) return NC_ERROR_INVALID_VALUE;
    const Variant *v = variant_of(name);
    if (!v) return NC_ERROR_NOT_FOUND;
    if (!v->dense) {
        if (capacity < 1) return NC_ERROR_INVALID_VALUE;
        params[0] = args;
        *count = 1;
        return NC_SUCCESS;
    }
    void *fields[] = {&args->q, &args->k, &args->v, &args->o, &args->seq_len, &args->head_dim, &args->q_stride,
                      &args->k_stride, &args->v_stride, &args->o_stride, &args->scale, &args->causal,
                      &args->q_row_stride, &args->k_row_stride, &args->v_row_stride, &args->o_row_stride,
                      &args->batch_heads, &args->num_q_blocks, &args->scratch, &args->balance_tail};
    static_assert(sizeof fields / sizeof fields[0] == NC_FLASH_MAX_KERNEL_PARAMS, "one parameter per field");
    if (capacity < NC_FLASH_MAX_KERNEL_PARAMS) return NC_ERROR_INVALID_VALUE;
    for (uint32_t i = 0; i < NC_FLASH_MAX_KERNEL_PARAMS; ++i) params[i] = fields[i];
    *count = NC_FLASH_MAX_KERNEL_PARAMS;
    return NC_SUCCESS;
}

int nc_flash_kernel_scratch_bytes(const char *name, const nc_flash_options *opts, uint64_t *bytes) {
    if (!name || !opts || !bytes) return NC_ERROR_INVALID_VALUE;
    *bytes = 0;
    for (const auto &v : kVariants)
        if (std::strcmp(v.name, name) == 0) {
            if (v.xsplit) {
                // one exchange counter per pair, and the counter region holds NC_XS_MAX_PAIRS
                if (xsplit_pairs(opts->batch_heads, opts->seq_len) > NC_XS_MAX_PAIRS)
                    return nc_internal_fail(NC_ERROR_INVALID_VALUE,
                                            "nc_flash_kernel_scratch_bytes: more pairs than NC_XS_MAX_PAIRS");
                *bytes = xsplit_scratch_bytes(opts->batch_heads, opts->seq_len, v.d);
            }
            return NC_SUCCESS;
        }
    return NC_ERROR_NOT_FOUND;
}

int nc_flash_reserve_workspace(nc_module module, const nc_flash_options *opts, void **workspace) {
    if (workspace) *workspace = nullptr;
    if (!module) return NC_ERROR_INVALID_VALUE;
    nc_flash_kernel_selection sel;
    int st = nc_flash_select_kernel(opts, &sel);
    if (st) return st;
    if (!sel.scratch_bytes) return NC_SUCCESS;
    void *ws = nullptr;
    st = nc_internal_module_workspace(module, sel.scratch_bytes, &ws);
    if (!st && workspace) *workspace = ws;
    return st;
}

int nc_flash_work_model(const nc_flash_options *opts, nc_flash_work *out) {
    if (!opts || !out) return NC_ERROR_INVALID_VALUE;
    const uint64_t bh = opts->batch_heads, s = opts->seq_len, d = opts->head_dim;
    const uint64_t eff = opts->causal ? (s * (s + 1)) / 2 : s * s;  // src/main.zig:1032
    out->flops_reference = bh * (4 * eff * d);                      // src/main.zig:1033
    out->flops_halfsquare = (4 * bh * s * s * d) / (opts->causal ? 2 : 1);
    out->bytes = bh * s * d * (2 * 3 + 4);                          // src/main.zig:1034
    return NC_SUCCESS;
}

}  // extern "C"
