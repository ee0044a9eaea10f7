// lal_gpu_sample.hip -- MI355X (gfx950) token sampler, int8 LM head and the
// C ABI declared in include/lal_gpu_sample.h.
//
// Sampling path (reference: runtime/lal_sampling.h:46-125,
// tools/server/qwen7b_server.c:219-295, tools/server/gpt2_server.c:2862-3012,
// compiler/lal.py:2218-2242).  One workgroup of four wave64s owns one row:
//
//   setup     history ids and ban ids go into an LDS hash (id -> occurrence
//             count, flags, exact processed logit); the exact value of every
//             history id is computed once from global memory.
//   stream    the row is read once with coalesced 16-byte loads, 8192 floats
//             per tile.  Each value gets its cheap upper bound (raw logit plus
//             bias, -inf when the allow bit is clear); values at or above the
//             running threshold tau look up the hash for their exact value
//             (repetition penalty and pre-selection bans only ever lower a
//             value) and are appended to an LDS candidate buffer.  When the
//             buffer would overflow, an LDS radix select over buffer + tile
//             raises tau to the k-th largest value seen so far, which can never
//             exceed the row's true k-th largest.
//   select    an LDS radix select over the buffer gives the exact k-th largest
//             value T (with multiplicity, as the reference's min-heap does).
//   epilogue  the candidates (value >= T) are sorted by id; nucleus (top-p),
//             lal_filter_topk bans, softmax and the inverse-CDF draw run over
//             them with the reference's sequential fp32 order and a bit-exact
//             restatement of glibc expf.
//
// When more than CAP logits tie at the threshold the buffer cannot hold the
// pool; the row is then finished by re-reading it in id order (rescan).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <climits>
#include <mutex>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "lal_gpq8.h"
#include "lal_gpu_sample.h"
#include "lal_gpu_workload.h"

namespace {

constexpr int WG = 256;             // threads per workgroup: 4 wave64
constexpr int NWAVE = WG / 64;
constexpr int U4 = 4;               // float4 loads per lane per wave-iteration
constexpr int VPL = 4 * U4;         // values per lane per wave-iteration
constexpr int WITER = 64 * U4;      // float4 per wave-iteration (1024 floats)
constexpr int HBITS = 10;
constexpr int HSLOTS = 1 << HBITS;  // LDS hash slots
constexpr int HCOUNT_MASK = 0xFFFF;
constexpr int HF_MASKPRE = 1 << 16; // id is -inf before selection
constexpr int HF_BAN = 1 << 17;     // id is dropped from the top-k pool
constexpr int EP_ALL = HSLOTS + NWAVE * 256;  // epilogue scratch floats (hval + histograms)
constexpr int RS_CHUNK = NWAVE * 256;         // rescan chunk (lives in the histogram area)
// per-wave candidate buffer entries: 512 when k <= 128, 2048 up to LAL_GPU_MAX_K
constexpr int CAPW_SMALL = 512;
constexpr int CAPW_LARGE = 1536;
constexpr int K_SMALL_MAX = 128;
constexpr int MAX_SLICES = 64;                 // slices per row
constexpr int FLAT_MAX = NWAVE * CAPW_LARGE;   // slice-list entries per row
constexpr int HMETA_STRIDE = 16;               // int4 per row of an LM head's list state (256 bytes)
constexpr int HSUB = 8;                        // sub-lists per row of an LM head's candidates
static_assert(HMETA_STRIDE >= 1 + HSUB, "list state: flags + sub-list counts");
// row sample for the threshold estimate: 64 float4 (1 KB) every SBLK float4
constexpr int SBLK = 2048;          // 32 KB stride -> 1/32 of the row
constexpr int SR = 5;               // float4 per thread: up to 20 sampled blocks (V <= 163840 fully sampled)

static_assert(2 * HSLOTS >= 3 * (LAL_GPU_MAX_HISTORY + LAL_GPU_MAX_BAN_IDS), "hash load <= 2/3");
static_assert(CAPW_SMALL > K_SMALL_MAX && CAPW_LARGE > LAL_GPU_MAX_K, "buffer above k");

// ---------------------------------------------------------------------------
// expf as glibc computes it (the reference calls glibc's expf).  This is the
// published algorithm of glibc 2.27+ / ARM optimized-routines e_expf.c:
// x*32/ln2 = k + r, 2^(k/32) from a 32-entry table, a cubic for 2^(r/32),
// evaluated in double.  The fused multiply-adds are the ones the x86-64 FMA
// build of glibc performs (the range reduction included); this restatement
// equals glibc expf on all 2^32 float inputs.
// ---------------------------------------------------------------------------
__constant__ uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

__device__ __forceinline__ float glibc_expf(float x, const uint64_t *tab)
{
    const uint32_t ux = __float_as_uint(x);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                     // |x| >= 88 or nan
        if (ux == 0xff800000u) return 0.0f;    // -inf
        if (abstop >= 0x7f8) return x + x;     // +inf or nan
        if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double InvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double Shift = 0x1.8p+52;
    const double C0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double C1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = __fma_rn(InvLn2N, xd, Shift);
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= Shift;
    const double r = __fma_rn(InvLn2N, xd, -kd);
    uint64_t t = tab[ki & 31];
    t += ki << 47;
    const double s = __longlong_as_double((long long)t);
    const double z = __fma_rn(C0, r, C1);
    const double r2 = r * r;
    double y = __fma_rn(C2, r, 1.0);
    y = __fma_rn(z, r2, y);
    y = y * s;
    return (float)y;
}

// Order-preserving float -> uint32 key (-0 folded onto +0; nan never enters).
__device__ __forceinline__ uint32_t fkey(float f)
{
    uint32_t u = __float_as_uint(f);
    if (u == 0x80000000u) u = 0;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float keyf(uint32_t k)
{
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// native vector types for the nontemporal 16-byte loads
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
// wave index as a wave-uniform (scalar) value
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Orders this wave's LDS accesses before/after the point (lanes of one wave
// exchange data through LDS without a workgroup barrier).
__device__ __forceinline__ void wave_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Wave64 scans and reductions with DPP row shifts and row broadcasts (VALU
// only, no LDS round trips): within each row of 16 lanes by row_shr 1, 2, 4,
// 8, then row 0's total into row 1 (row_bcast:15, rows 1 and 3) and rows 0-1's
// total into rows 2-3 (row_bcast:31).  Lanes without a source keep `old`, the
// identity.  Reductions return lane 63's value (uniform).
#define LAL_DPP_SCAN(OP, T, IDENT, TOI, FROMI)                                            \
    do {                                                                                  \
        v = OP(v, FROMI(__builtin_amdgcn_update_dpp(TOI(IDENT), TOI(v), 0x111, 0xf, 0xf, false))); \
        v = OP(v, FROMI(__builtin_amdgcn_update_dpp(TOI(IDENT), TOI(v), 0x112, 0xf, 0xf, false))); \
        v = OP(v, FROMI(__builtin_amdgcn_update_dpp(TOI(IDENT), TOI(v), 0x114, 0xf, 0xf, false))); \
        v = OP(v, FROMI(__builtin_amdgcn_update_dpp(TOI(IDENT), TOI(v), 0x118, 0xf, 0xf, false))); \
        v = OP(v, FROMI(__builtin_amdgcn_update_dpp(TOI(IDENT), TOI(v), 0x142, 0xa, 0xf, false))); \
        v = OP(v, FROMI(__builtin_amdgcn_update_dpp(TOI(IDENT), TOI(v), 0x143, 0xc, 0xf, false))); \
    } while (0)

__device__ __forceinline__ int op_add(int a, int b) { return a + b; }
__device__ __forceinline__ int op_min(int a, int b) { return min(a, b); }
__device__ __forceinline__ unsigned op_maxu(unsigned a, unsigned b) { return max(a, b); }
__device__ __forceinline__ unsigned op_minu(unsigned a, unsigned b) { return min(a, b); }
__device__ __forceinline__ float op_fmax(float a, float b) { return fmaxf(a, b); }
__device__ __forceinline__ int id_i(int x) { return x; }
__device__ __forceinline__ int u2i(unsigned x) { return (int)x; }
__device__ __forceinline__ unsigned i2u(int x) { return (unsigned)x; }
__device__ __forceinline__ int f2i(float x) { return __float_as_int(x); }
__device__ __forceinline__ float i2f(int x) { return __int_as_float(x); }

__device__ __forceinline__ int wave_incl_scan(int v)
{
    LAL_DPP_SCAN(op_add, int, 0, id_i, id_i);
    return v;
}

__device__ __forceinline__ float wave_max(float v)
{
    LAL_DPP_SCAN(op_fmax, float, -INFINITY, f2i, i2f);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ int wave_min(int v)
{
    LAL_DPP_SCAN(op_min, int, INT_MAX, id_i, id_i);
    return __builtin_amdgcn_readlane(v, 63);
}

__device__ __forceinline__ int wave_sum(int v)
{
    LAL_DPP_SCAN(op_add, int, 0, id_i, id_i);
    return __builtin_amdgcn_readlane(v, 63);
}

__device__ __forceinline__ unsigned wave_max_u(unsigned v)
{
    LAL_DPP_SCAN(op_maxu, unsigned, 0u, u2i, i2u);
    return (unsigned)__builtin_amdgcn_readlane((int)v, 63);
}

__device__ __forceinline__ unsigned wave_min_u(unsigned v)
{
    LAL_DPP_SCAN(op_minu, unsigned, 0xFFFFFFFFu, u2i, i2u);
    return (unsigned)__builtin_amdgcn_readlane((int)v, 63);
}

__device__ __forceinline__ int readlane_i(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ float readlane_f(float v, int l)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Device-coherent (agent-scope) plain accesses, for data exchanged between
// workgroups of one launch.
template <class T>
__device__ __forceinline__ void dev_store(T *p, T v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ T dev_load(const T *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until this thread's outstanding memory operations have completed.
__device__ __forceinline__ void wait_stores_done() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <int CAPW>
struct Smem {
    float cval[NWAVE * CAPW];  // per-wave candidate buffers: exact processed logits
    int cidx[NWAVE * CAPW];    // ... and their token ids
    int hkey[HSLOTS];          // hash: token id or -1
    int hinfo[HSLOTS];         // occurrence count | HF_* flags
    union {
        struct {
            float hval[HSLOTS];            // exact processed logit of the id
            unsigned whist[NWAVE][256];    // per-wave radix histograms
        } h;
        float ep[EP_ALL];                  // epilogue scratch (after streaming)
    } u;
    int wcnt[NWAVE];      // entries in each wave buffer (dead ones are nan)
    int walive[NWAVE];    // live entries
    unsigned tau_key;     // max over the waves' thresholds (order-preserving key)
    int nan_flag;         // the row holds a nan processed value
    unsigned bias_key;    // key of the largest flagged bias entry (all ones: a nan or -inf)
    float wtau[NWAVE];
    int wstrict[NWAVE];
    int wsum[2][NWAVE];
    float redf[NWAVE];
    int redi[NWAVE];
    int redi2[NWAVE];
    int sel_digit;
    int sel_rem;
    int gcount;           // keys gathered by the select's final step
    unsigned wkmax[NWAVE];  // per-wave range of the live buffer keys
    unsigned wkmin[NWAVE];
    uint64_t exptab[32];  // glibc's 2^(i/32) table (LDS copy of kExp2Tab)
};

struct KArgs {
    const float *logits;
    float *logits_w;
    int ld, V;
    const int *hist;
    int hist_ld;
    const int *hist_len;
    const uint32_t *allow;
    int allow_ld;
    const float *bias;
    const uint32_t *bias_bits;  // bit e set unless bias[e] is +0.0 (bias_prep_kernel)
    const uint32_t *bias_part;  // per-block maximum keys of the flagged bias entries
    int bias_nparts;            // <= WG
    const float *uniforms;
    int *out_token;
    float *out_thr;
    int *out_ncand;
    int *out_nkept;
    float *out_sum;
    int cand_ld;
    int *cand_ids;
    float *cand_probs;
    uint8_t *cand_kept;
    float *cand_vals;
    float *out_hvals;
    const int *ban_ids;
    int n_ban;
    const int *last_tokens;  // [batch] id ban_last drops (NULL: history[len-1])
    float T, top_p, pen;
    int k;
    int variant;
    unsigned flags;
    int ban_last, ban_repeat, mask_recent;
    int greedy;     // greedy path: k = 1, first index among the maxima
    int fallback;   // token when no running sum reaches r: V-1, or 0 (F_FALLBACK_ZERO)
    int apply_pen;  // penalty applied for this variant / greedy state
    int any_bans;
    // slicing: each row is split into nslice contiguous slices, one workgroup
    // each; a slice publishes its candidates (at most lcap) and the last slice
    // to arrive finishes the row
    int batch;
    int nslice;
    int lcap;
    float *lst_val;     // [batch][nslice][lcap] candidate values
    int *lst_idx;       // [batch][nslice][lcap] candidate ids
    int4 *lst_meta;     // [batch][nslice] (count, threshold bits, strict, -)
    unsigned *arrive;   // [batch] slices finished; reset by the finisher
    // candidate lists an LM head wrote (list mode): row b's entries at
    // lst_val / lst_idx + b * hcap in HSUB sub-lists of hcap / HSUB entries,
    // hmeta[b * HMETA_STRIDE] = (-, -, -, flags: 1 list full, 2 a nan logit),
    // hmeta[b * HMETA_STRIDE + 1 + s].x = entries of sub-list s, hslots[b][64]
    // the sample slots the bound comes from (rank hks); both are cleared by
    // the row's workgroup for the next head
    int4 *hmeta;
    unsigned *hslots;
    int hcap;
    int hks;            // rank of the head's bound among the 64 slots
    int prio_rotate;    // rotate the stream's wave priority over the CU's four workgroups
    int ncu;            // compute units: workgroups [3*ncu, 4*ncu) are the
                        // fourth (youngest) resident on their CU
};

// block reductions (barriers inside; callers keep control flow uniform)
template <class SM>
__device__ __forceinline__ float block_max(SM &S, float v)
{
    v = wave_max(v);
    __syncthreads();
    if (lane_id() == 0) S.redf[wave_id()] = v;
    __syncthreads();
    float r = S.redf[0];
#pragma unroll
    for (int w = 1; w < NWAVE; ++w) r = fmaxf(r, S.redf[w]);
    return r;
}

template <class SM>
__device__ __forceinline__ int block_min(SM &S, int v)
{
    v = wave_min(v);
    __syncthreads();
    if (lane_id() == 0) S.redi[wave_id()] = v;
    __syncthreads();
    int r = S.redi[0];
#pragma unroll
    for (int w = 1; w < NWAVE; ++w) r = min(r, S.redi[w]);
    return r;
}

template <class SM>
__device__ __forceinline__ int block_sum(SM &S, int v)
{
    v = wave_sum(v);
    __syncthreads();
    if (lane_id() == 0) S.redi2[wave_id()] = v;
    __syncthreads();
    int r = 0;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) r += S.redi2[w];
    return r;
}

// exclusive block scan; one barrier; wsum must alternate between calls
__device__ __forceinline__ int block_excl_scan(int v, int &total, int *wsum)
{
    const int incl = wave_incl_scan(v);
    if (lane_id() == 63) wsum[wave_id()] = incl;
    __syncthreads();
    int before = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
        const int s = wsum[w];
        before += (w < wave_id()) ? s : 0;
        tot += s;
    }
    total = tot;
    return before + incl - v;
}

// ---------------------------------------------------------------------------
// LDS hash of the row's history / ban ids
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t hslot(int key)
{
    return ((uint32_t)key * 2654435761u) >> (32 - HBITS);
}

__device__ __forceinline__ void hash_insert(int *hkey, int *hinfo, int key, int add, int flags)
{
    uint32_t s = hslot(key);
    for (int probe = 0; probe < HSLOTS; ++probe) {
        const int prev = atomicCAS(&hkey[s], -1, key);
        if (prev == -1 || prev == key) {
            if (add) atomicAdd(&hinfo[s], add);
            if (flags) atomicOr(&hinfo[s], flags);
            return;
        }
        s = (s + 1) & (HSLOTS - 1);
    }
}

__device__ __forceinline__ int hash_find(const int *hkey, int key)
{
    uint32_t s = hslot(key);
    for (int probe = 0; probe < HSLOTS; ++probe) {
        const int k = hkey[s];
        if (k == key) return (int)s;
        if (k == -1) return -1;
        s = (s + 1) & (HSLOTS - 1);
    }
    return -1;
}

__device__ __forceinline__ bool allow_bit(const uint32_t *row_bits, int e)
{
    return (row_bits[e >> 5] >> (e & 31)) & 1u;
}

// repetition penalty applied `count` times: x>0 ? x/p : x*p
// (runtime/lal_sampling.h:63-64, once per history occurrence).  A nan stays
// the same nan, bit for bit, as the x86 multiply returns it.
__device__ __forceinline__ float penalise(float x, int count, float pen)
{
    if (x != x) return x;
    for (int c = 0; c < count; ++c) x = (x > 0.0f) ? x / pen : x * pen;
    return x;
}

__device__ __forceinline__ bool passes(float y, float tau, bool strict)
{
    return strict ? (y > tau) : (y >= tau);
}

// Smallest float above t (y > t  <=>  y >= next_up(t) for non-nan y); +inf
// maps to nan so that nothing passes.
__device__ __forceinline__ float next_up(float t)
{
    const uint32_t u = __float_as_uint(t);
    if (t != t || u == 0x7f800000u) return __uint_as_float(0x7fc00000u);
    if ((u & 0x7fffffffu) == 0) return __uint_as_float(1u);  // +-0 -> smallest denormal
    return __uint_as_float((u & 0x80000000u) ? u - 1 : u + 1);
}

// Sequential fp32 prefix sums over ep[0..n) in index order, done by wave 0
// (lane l of a 64-chunk receives the running sum after element base+l).  The
// additions happen in exactly the order of the reference's scalar loop.
// Entries < 0 mark "not in the set" and are skipped.  Writes the inclusive
// prefix back into ep and returns the total to every thread.
template <class SM>
__device__ __forceinline__ float block_seq_prefix(SM &S, float *ep, int n, float carry_in)
{
    __syncthreads();
    if (wave_id() == 0) {
        float acc = carry_in;
        const int me = lane_id();
        for (int base = 0; base < n; base += 64) {
            const int i = base + me;
            float e = (i < n) ? ep[i] : -1.0f;
            const unsigned long long live = __ballot(!(e < 0.0f));
            float pre = acc;
            if (live) {
                // a skipped entry (< 0, and the lanes past n) adds -0.0, which
                // leaves every sum as it is (x + -0.0 == x, also for +0.0 and
                // -0.0), so the chain is one add per entry, fully unrolled
                e = (e < 0.0f) ? -0.0f : e;
#pragma unroll
                for (int l = 0; l < 64; ++l) {
                    acc = acc + readlane_f(e, l);
                    if (me == l) pre = acc;
                }
            }
            if (i < n) ep[i] = pre;
        }
        if (lane_id() == 0) S.redf[0] = acc;
    }
    __syncthreads();
    const float tot = S.redf[0];
    __syncthreads();
    return tot;
}

// Inclusive sequential prefix over the lanes of one wave (lane order), values
// < 0 skipped; returns this lane's running sum, *total the sum over all lanes.
__device__ __forceinline__ float wave_seq_prefix(float e, int n, float *total)
{
    float acc = 0.0f, pre = 0.0f;
    const int me = lane_id();
    for (int l = 0; l < n; ++l) {
        const float el = readlane_f(e, l);
        if (!(el < 0.0f)) acc = acc + el;
        if (me == l) pre = acc;
    }
    *total = acc;
    return pre;
}

// ---------------------------------------------------------------------------
// Element addressing for a row: [0, head) scalar head elements, then nb4
// aligned float4 chunks, then a scalar tail of < 4 elements.
// ---------------------------------------------------------------------------
struct RowGeo {
    int head, nb4, tail0, ntail;
};

__device__ __forceinline__ RowGeo row_geo(const float *row, int V)
{
    RowGeo g;
    const int mis = (int)(((uintptr_t)row >> 2) & 3);
    g.head = min((4 - mis) & 3, V);
    g.nb4 = (V - g.head) >> 2;
    g.tail0 = g.head + 4 * g.nb4;
    g.ntail = V - g.tail0;
    return g;
}

__device__ __forceinline__ int extra_elem(const RowGeo &g, int t)
{
    if (t < g.head) return t;
    if (t < g.head + g.ntail) return g.tail0 + (t - g.head);
    return -1;
}

// Bits [rel, rel + 4) of a bitmap window spread over the wave, one word per
// lane (lane i: word i); two words when the bits may straddle a word edge.
__device__ __forceinline__ uint32_t window_nibble(uint32_t word, int rel, bool two)
{
    const int wi = rel >> 5;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute(wi << 2, (int)word);
    if (!two) return (lo >> (rel & 31)) & 0xFu;
    const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute((wi + 1) << 2, (int)word);
    return (uint32_t)((((uint64_t)hi << 32) | lo) >> (rel & 31)) & 0xFu;
}

// cheap upper bound of the processed logit: raw + bias, -inf if not allowed
template <bool HAS_BIAS, bool HAS_ALLOW>
__device__ __forceinline__ float upper_bound(const float *bias, const uint32_t *abits, int e, float x)
{
    float y = x;
    if (HAS_BIAS) y = y + bias[e];
    if (HAS_ALLOW) {
        if (!allow_bit(abits, e)) y = -INFINITY;
    }
    return y;
}

// Exact processed value of token e given its upper bound yhat: ids in the
// hash are recomputed from the raw logit (penalty applied `count` times, then
// bias, allow mask and the pre-selection ban); all others equal the bound.
struct RowCtx {
    const float *row;
    const float *bias;
    const uint32_t *abits;
    const int *hkey;
    const int *hinfo;
    float pen;
    bool has_bias, has_allow, use_hash;
    bool bound_bias;  // bounds may carry the bias maximum in place of bias[e]
    const uint32_t *bias_bits;  // ... for the ids whose bit is set here
};

// exact value of id e from its upper bound yhat, given its hash slot s (-1:
// not in the hash, and the bound is exact unless it may carry the bias
// maximum)
__device__ __forceinline__ float exact_at_slot(const RowCtx &R, int e, float yhat, int s)
{
    // outside the hash the bound is exact unless it carries the bias maximum
    // (the id's bias bit is set; the map is small and cached, the row is not)
    if (s < 0 && (!R.bound_bias || !((R.bias_bits[e >> 5] >> (e & 31)) & 1u))) return yhat;
    const int info = (s >= 0) ? R.hinfo[s] : 0;
    // without a bias the upper bound is the raw logit (or -inf when the allow
    // bit is clear, which the mask below keeps)
    const float raw = R.has_bias ? R.row[e] : yhat;
    float y = penalise(raw, info & HCOUNT_MASK, R.pen);
    if (R.has_bias) y = y + R.bias[e];
    if (R.has_allow && !allow_bit(R.abits, e)) y = -INFINITY;
    if (info & HF_MASKPRE) y = -INFINITY;
    return y;
}

__device__ __forceinline__ float exact_value(const RowCtx &R, int e, float yhat)
{
    return exact_at_slot(R, e, yhat, R.use_hash ? hash_find(R.hkey, e) : -1);
}

// k-th largest of the 64 lane keys (1 <= k <= 64), bit by bit: the largest K
// with at least k keys >= K.  Ballot counts only; wave-synchronous.
__device__ __forceinline__ uint32_t wave_kth_lane_key(uint32_t key, int k)
{
    uint32_t K = 0u;
    for (int bit = 31; bit >= 0; --bit) {
        const uint32_t cand = K | (1u << bit);
        if (__popcll(__ballot(key >= cand)) >= k) K = cand;
    }
    return K;
}

// ---------------------------------------------------------------------------
// Per-wave state and candidate buffer
// ---------------------------------------------------------------------------
struct WState {
    float tau;   // running lower bound of the row's k-th largest processed logit
    int strict;  // 1: buffer holds values > tau (more than CAPW tie at tau)
    int cnt;     // entries in the wave's buffer
    float tcmp;  // the wave's own filter: values >= tcmp pass (next_up(tau)
                 // when strict; nan, which nothing passes, above +inf)
};

// Wave radix select: k-th largest key over bv[0..cnt) and the lanes' values
// y[i] with bit i of m set.  Requires >= k inputs.  Wave-synchronous.
template <int NV>
__device__ __forceinline__ uint32_t wave_kth_key(unsigned *hist, const float *bv, int cnt,
                                                 const float (&y)[NV], uint32_t m, int k)
{
    uint32_t prefix = 0, pmask = 0;
    int rem = k;
    const int lane = lane_id();
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        hist[4 * lane + 0] = 0;
        hist[4 * lane + 1] = 0;
        hist[4 * lane + 2] = 0;
        hist[4 * lane + 3] = 0;
        wave_sync();
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            if ((m >> i) & 1u) {
                const uint32_t key = fkey(y[i]);
                if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
            }
        }
        for (int j = lane; j < cnt; j += 64) {
            const float v = bv[j];
            if (v != v) continue;
            const uint32_t key = fkey(v);
            if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
        }
        wave_sync();
        const int b0 = 255 - 4 * lane;
        const int h0 = hist[b0], h1 = hist[b0 - 1], h2 = hist[b0 - 2], h3 = hist[b0 - 3];
        const int lsum = h0 + h1 + h2 + h3;
        const int incl = wave_incl_scan(lsum);
        const int excl = incl - lsum;
        const bool hit = (excl < rem && rem <= incl);
        int r = rem - excl, d = b0;
        if (r <= h0) d = b0;
        else if ((r -= h0) <= h1) d = b0 - 1;
        else if ((r -= h1) <= h2) d = b0 - 2;
        else { r -= h2; d = b0 - 3; }
        const unsigned long long hm = __ballot(hit);
        const int src = hm ? (int)__builtin_ctzll(hm) : 0;
        d = readlane_i(d, src);
        r = readlane_i(r, src);
        prefix |= (uint32_t)d << shift;
        pmask |= 0xFFu << shift;
        rem = r;
        wave_sync();
    }
    return prefix;
}

// Buffer entries whose id carries UNREFINED hold the cheap upper bound (raw
// logit + bias, allow mask applied); their exact value (penalty, pre-selection
// bans) is looked up only when the wave must select or at the end.  A refined
// entry that fails the current threshold becomes dead (value nan).
constexpr int UNREFINED = (int)0x80000000;

__device__ __forceinline__ void wave_refine(float *bv, int *bi, int cnt, const RowCtx &R, float tau,
                                            bool strict)
{
    for (int j = lane_id(); j < cnt; j += 64) {
        const int id = bi[j];
        if (!(id & UNREFINED)) continue;
        const int e = id & ~UNREFINED;
        const float y = exact_value(R, e, bv[j]);
        bv[j] = passes(y, tau, strict) ? y : NAN;
        bi[j] = e;
    }
    wave_sync();
}

// wave_refine for the end of the stream, when the stream's registers are
// free (inside the stream loop the extra registers would spill).
__device__ __forceinline__ void wave_refine_batched(float *bv, int *bi, int cnt, const RowCtx &R, float tau,
                                                    bool strict)
{
    // eight entries per lane at a time: their buffer reads, then their first
    // hash probes, are in flight together (linear probing rarely goes on)
    constexpr int RB = 8;
    const int lane = lane_id();
    for (int j0 = 0; j0 < cnt; j0 += RB * 64) {
        int id[RB], slot[RB], key[RB];
        float yh[RB];
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int j = j0 + r * 64 + lane;
            id[r] = (j < cnt) ? bi[j] : 0;
            yh[r] = (j < cnt) ? bv[j] : NAN;
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            slot[r] = (int)hslot(id[r] & ~UNREFINED);
            key[r] = (id[r] & UNREFINED) ? R.hkey[slot[r]] : -1;
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            if (!(id[r] & UNREFINED)) continue;
            const int e = id[r] & ~UNREFINED;
            int sl = slot[r], k = key[r];
            for (int probe = 1; probe < HSLOTS && k != e && k != -1; ++probe) {
                sl = (sl + 1) & (HSLOTS - 1);
                k = R.hkey[sl];
            }
            const float y = exact_at_slot(R, e, yh[r], k == e ? sl : -1);
            const int j = j0 + r * 64 + lane;
            bv[j] = passes(y, tau, strict) ? y : NAN;
            bi[j] = e;
        }
    }
    wave_sync();
}

// Offer this wave's values to its buffer.  x[i] are upper bounds whose pass
// bit is set in m.  On overflow the wave refines its buffer and the offered
// values, raises tau to the k-th largest of them and compacts.
// Wave-synchronous, no workgroup barrier.
__device__ __forceinline__ int lanes_below(unsigned long long mk)
{
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mk >> 32),
                                          __builtin_amdgcn_mbcnt_lo((uint32_t)mk, 0u));
}

// In-place compaction of bv/bi[0..cnt) keeping entries that pass (tau,
// strict), 64 entries at a time (every lane reads its entry before any lane
// writes, and writes never reach an entry not yet read).  Returns the count.
__device__ __forceinline__ int wave_compact(float *bv, int *bi, int cnt, float tau, bool strict)
{
    int base = 0;
    const int lane = lane_id();
    for (int j0 = 0; j0 < cnt; j0 += 64) {
        const int j = j0 + lane;
        const float v = (j < cnt) ? bv[j] : NAN;
        const int id = (j < cnt) ? bi[j] : 0;
        const bool keep = passes(v, tau, strict);
        const unsigned long long mk = __ballot(keep);
        if (keep) {
            const int pos = base + lanes_below(mk);
            bv[pos] = v;
            bi[pos] = id;
        }
        base += __popcll(mk);
    }
    wave_sync();
    return base;
}

// Append the offered values x[i] (bit i of m) that pass (tau, strict).
template <int NQ>
__device__ __forceinline__ int wave_append(float *bv, int *bi, int base, const float (&x)[4 * NQ],
                                           const int (&eb)[NQ], uint32_t m, float tau, bool strict,
                                           int tag)
{
#pragma unroll
    for (int i = 0; i < 4 * NQ; ++i) {
        const bool p = ((m >> i) & 1u) && passes(x[i], tau, strict);
        const unsigned long long mk = __ballot(p);
        if (mk) {
            if (p) {
                const int pos = base + lanes_below(mk);
                bv[pos] = x[i];
                bi[pos] = (eb[i >> 2] + (i & 3)) | tag;
            }
            base += __popcll(mk);
        }
    }
    return base;
}

// Offer this wave's values to its buffer: x[i] are upper bounds of the
// processed logits (nan when out of range), tcmp the current filter.  On
// overflow the wave resolves exact values (into a separate array), raises tau
// to the k-th largest of buffer + offered values and compacts.  pm[i] is the
// caller's ballot of x[i] >= tcmp: the masks come in as scalar values, so the
// compiler never holds the comparisons as per-lane booleans across the call.
// Wave-synchronous, no workgroup barrier.
template <int NQ, int CAPW>
__device__ __forceinline__ void wave_offer(float *bv, int *bi, unsigned *hist, const RowCtx &R,
                                           const float (&x)[4 * NQ], const unsigned long long (&pm)[4 * NQ],
                                           const int (&eb)[NQ], float tcmp, WState &st, int k,
                                           unsigned *tau_key_shared)
{
    constexpr int NV = 4 * NQ;
    const int tag = (R.use_hash || R.bound_bias) ? UNREFINED : 0;
    // append path: the per-slot ballots give the count (scalar popcounts) and
    // each lane's position (mbcnt); no cross-lane data exchange
    int total = 0;
#pragma unroll
    for (int i = 0; i < NV; ++i) total += __popcll(pm[i]);
    if (total == 0) return;
    // the lanes' own tests go through an opaque copy of the filter, so that
    // they are not merged with the caller's ballots
    float tl = tcmp;
    asm volatile("" : "+v"(tl));
    if (st.cnt + total <= CAPW) {
        int base = st.cnt;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const unsigned long long mk = pm[i];
            if (mk) {
                if (x[i] >= tl) {
                    const int pos = base + lanes_below(mk);
                    bv[pos] = x[i];
                    bi[pos] = (eb[i >> 2] + (i & 3)) | tag;
                }
                base += __popcll(mk);
            }
        }
        st.cnt = base;
        return;
    }
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < NV; ++i) m |= (x[i] >= tl) ? (1u << i) : 0u;
    // overflow: exact values for the offered entries and the buffer
    float y[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        y[i] = x[i];
        if ((m >> i) & 1u) {
            y[i] = exact_value(R, eb[i >> 2] + (i & 3), x[i]);
            if (!passes(y[i], st.tau, st.strict)) m &= ~(1u << i);
        }
    }
    wave_sync();
    if (R.use_hash || R.bound_bias) wave_refine(bv, bi, st.cnt, R, st.tau, st.strict);
    int cnt = wave_compact(bv, bi, st.cnt, st.tau, st.strict);
    const int offered = wave_sum(__popc(m));
    float tk = st.tau;
    bool strict = st.strict;
    if (cnt + offered > CAPW) {
        // count of buffer + offered values >= t
        auto count_ge = [&](float t) {
            int nge = 0;
            for (int j = lane_id(); j < cnt; j += 64) nge += (bv[j] >= t);
#pragma unroll
            for (int i = 0; i < NV; ++i) nge += ((m >> i) & 1u) && (y[i] >= t);
            return wave_sum(nge);
        };
        int nge = CAPW + 1;
        if (k <= 64) {
            // The k-th largest of the lanes' maxima: k distinct values of the
            // set reach it, so it is no larger than the set's k-th largest (a
            // valid, cheap bound).  Used only when it leaves at most CAPW
            // values: strictly above it there can be more than CAPW (up to k-1
            // lanes' worth), and a lane without values makes it key 0.
            uint32_t mk = 0u;
#pragma unroll
            for (int i = 0; i < NV; ++i)
                if ((m >> i) & 1u) mk = max(mk, fkey(y[i]));
            for (int j = lane_id(); j < cnt; j += 64) {
                const float v = bv[j];
                if (v == v) mk = max(mk, fkey(v));
            }
            const uint32_t K = wave_kth_lane_key(mk, k);
            if (K != 0u) {
                tk = keyf(K);
                nge = count_ge(tk);
            }
        }
        if (nge > CAPW) {
            // the exact k-th largest: fewer than k <= CAPW values lie above it
            tk = keyf(wave_kth_key<NV>(hist, bv, cnt, y, m, k));
            nge = count_ge(tk);
        }
        strict = nge > CAPW;
        cnt = wave_compact(bv, bi, cnt, tk, strict);
    }
    st.cnt = wave_append<NQ>(bv, bi, cnt, y, eb, m, tk, strict, 0);
    wave_sync();
    if (tk != st.tau || strict != (bool)st.strict) {
        st.tau = tk;
        st.strict = strict ? 1 : 0;
        st.tcmp = strict ? next_up(tk) : tk;
        if (lane_id() == 0) atomicMax(tau_key_shared, fkey(tk));
    }
}

// Range of the live buffer keys over the block, from the per-wave ranges the
// waves stored in S.wkmax / S.wkmin (0 / 0xFFFFFFFF for none).
template <class SM>
__device__ __forceinline__ void block_key_range(const SM &S, uint32_t &kmin, uint32_t &kmax)
{
    kmax = 0u;
    kmin = 0xFFFFFFFFu;
#pragma unroll
    for (int ww = 0; ww < NWAVE; ++ww) {
        kmax = max(kmax, (uint32_t)S.wkmax[ww]);
        kmin = min(kmin, (uint32_t)S.wkmin[ww]);
    }
}

// Block radix select over the union of the wave buffers (each thread reads
// its own wave's entries).  Requires >= k entries in total; kmin / kmax is the
// range of the live keys (block_key_range).  The bits above the highest one
// where kmin and kmax differ are common; the rest go 8 per pass with one
// barrier each (three histograms in rotation, and every wave derives the
// digit itself).  Once the chosen bin holds at most 64 keys they are gathered
// and every wave ranks them directly.  Every thread calls it; no barrier is
// needed after it before the wave buffers or S.wsum are written again.
template <int CAPW, class SM>
__device__ __forceinline__ uint32_t block_kth_union(SM &S, int k, uint32_t kmin, uint32_t kmax)
{
    constexpr int PK = CAPW / 64;  // entries per lane of its own wave's buffer
    if (kmin >= kmax) return kmax;  // every live key is equal (k <= count)
    const int w = wave_id(), lane = lane_id();
    const int cnt = S.wcnt[w];
    const float *bv = S.cval + w * CAPW;
    // keys of the live entries (0 = none); reads stay inside the wave's buffer
    uint32_t key[PK];
#pragma unroll
    for (int r = 0; r < PK; ++r) {
        const int j = lane + 64 * r;
        const float v = bv[j];
        key[r] = (j < cnt && v == v) ? fkey(v) : 0u;
    }
    S.u.h.whist[0][threadIdx.x] = 0;
    S.u.h.whist[1][threadIdx.x] = 0;
    S.u.h.whist[3][threadIdx.x] = 0;  // gather slots (see the final step)
    if (threadIdx.x == 0) S.gcount = 0;
    __syncthreads();
    const int L = __builtin_clz(kmin ^ kmax);
    uint32_t pmask = L ? ~0u << (32 - L) : 0u;
    uint32_t prefix = kmax & pmask;
    int rem = k;
    int p = 0;
    for (int hi = 31 - L; hi >= 0; hi -= 8, ++p) {
        unsigned *hist = S.u.h.whist[p % 3];
        const int lo = max(hi - 7, 0);
        const uint32_t dmask = (hi - lo == 31) ? ~0u : ((1u << (hi - lo + 1)) - 1u);
#pragma unroll
        for (int r = 0; r < PK; ++r)
            if (key[r] && (key[r] & pmask) == prefix) atomicAdd(&hist[(key[r] >> lo) & dmask], 1u);
        // the next pass's histogram was last read before the previous barrier
        S.u.h.whist[(p + 1) % 3][threadIdx.x] = 0;
        __syncthreads();
        const int b0 = 255 - 4 * lane;
        const int h0 = hist[b0], h1 = hist[b0 - 1], h2 = hist[b0 - 2], h3 = hist[b0 - 3];
        const int lsum = h0 + h1 + h2 + h3;
        const int incl = wave_incl_scan(lsum);
        const int excl = incl - lsum;
        const bool hit = (excl < rem && rem <= incl);
        int r = rem - excl, d = b0, hb = h0;
        if (r <= h0) { d = b0; hb = h0; }
        else if ((r -= h0) <= h1) { d = b0 - 1; hb = h1; }
        else if ((r -= h1) <= h2) { d = b0 - 2; hb = h2; }
        else { r -= h2; d = b0 - 3; hb = h3; }
        const unsigned long long hm = __ballot(hit);
        const int src = hm ? (int)__builtin_ctzll(hm) : 0;
        d = readlane_i(d, src);
        r = readlane_i(r, src);
        hb = readlane_i(hb, src);
        prefix |= (uint32_t)d << lo;
        pmask |= dmask << lo;
        rem = r;
        if (lo > 0 && hb <= 64) {
            // few keys left with this prefix: gather them and rank directly
            unsigned *gk = S.u.h.whist[3];
#pragma unroll
            for (int r2 = 0; r2 < PK; ++r2)
                if (key[r2] && (key[r2] & pmask) == prefix) gk[atomicAdd(&S.gcount, 1)] = key[r2];
            __syncthreads();
            // slots past hb hold 0 (cleared at the start), below every
            // live key: the loop covers only the gathered quads
            const uint32_t mine = (lane < hb) ? gk[lane] : 0u;
            int gt = 0, ge = 0;
            for (int q = 0; q < ((hb + 3) >> 2); ++q) {
                const uint4 v4 = reinterpret_cast<const uint4 *>(gk)[q];
                gt += (v4.x > mine) + (v4.y > mine) + (v4.z > mine) + (v4.w > mine);
                ge += (v4.x >= mine) + (v4.y >= mine) + (v4.z >= mine) + (v4.w >= mine);
            }
            const unsigned long long fm = __ballot(lane < hb && gt < rem && rem <= ge);
            return (uint32_t)readlane_i((int)mine, fm ? (int)__builtin_ctzll(fm) : 0);
        }
    }
    return prefix;
}

// Block radix select: k-th largest key over the register values v[i] of all
// threads whose bit is set in m.  Requires >= k inputs.
template <int NV, class SM>
__device__ __forceinline__ uint32_t block_kth_regs(SM &S, const float (&v)[NV], uint32_t m, int k)
{
    unsigned *hist = S.u.h.whist[0];
    uint32_t prefix = 0, pmask = 0;
    int rem = k;
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        __syncthreads();
        hist[threadIdx.x] = 0;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            if ((m >> i) & 1u) {
                const uint32_t key = fkey(v[i]);
                if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
            }
        }
        __syncthreads();
        if (wave_id() == 0) {
            const int lane = lane_id();
            const int b0 = 255 - 4 * lane;
            const int h0 = hist[b0], h1 = hist[b0 - 1], h2 = hist[b0 - 2], h3 = hist[b0 - 3];
            const int lsum = h0 + h1 + h2 + h3;
            const int incl = wave_incl_scan(lsum);
            const int excl = incl - lsum;
            if (excl < rem && rem <= incl) {
                int r = rem - excl, d;
                if (r <= h0) d = b0;
                else if ((r -= h0) <= h1) d = b0 - 1;
                else if ((r -= h1) <= h2) d = b0 - 2;
                else { r -= h2; d = b0 - 3; }
                S.sel_digit = d;
                S.sel_rem = r;
            }
        }
        __syncthreads();
        prefix |= (uint32_t)S.sel_digit << shift;
        pmask |= 0xFFu << shift;
        rem = S.sel_rem;
    }
    __syncthreads();
    return prefix;
}

// ---------------------------------------------------------------------------
// Rescan path: finish the row by re-reading it in id order (used when more
// tokens tie at the threshold than the buffers hold).
// ---------------------------------------------------------------------------
template <bool HAS_BIAS, bool HAS_ALLOW, class SM>
__device__ __forceinline__ float rescan_value(const KArgs &A, const SM &S, const float *row,
                                              const uint32_t *abits, bool use_hash, int e)
{
    const float yh = upper_bound<HAS_BIAS, HAS_ALLOW>(A.bias, abits, e, row[e]);
    RowCtx R;
    R.row = row;
    R.bias = A.bias;
    R.abits = abits;
    R.hkey = S.hkey;
    R.hinfo = S.hinfo;
    R.pen = A.pen;
    R.has_bias = HAS_BIAS;
    R.has_allow = HAS_ALLOW;
    R.use_hash = use_hash;
    R.bound_bias = false;
    return exact_value(R, e, yh);
}

template <class SM>
__device__ __forceinline__ bool is_banned(const SM &S, int e)
{
    const int s = hash_find(S.hkey, e);
    return s >= 0 && (S.hinfo[s] & HF_BAN);
}

// The top-p nucleus of a rescanned row (gpt2_server.c:2908-2955): in the
// order (probability desc, id asc) the kept tokens are a prefix, so the set is
// {p > plim} plus {p == plim and id <= idlim}, p = expf((y - amax)/T) * inv.
struct Nucleus {
    bool on;
    float amax, inv, plim;
    int idlim;
};

template <class SM>
__device__ __forceinline__ bool in_nucleus(const KArgs &A, const SM &S, const Nucleus &N, float y,
                                           int e)
{
    if (!N.on) return true;
    const float p = glibc_expf((y - N.amax) / A.T, S.exptab) * N.inv;
    return p > N.plim || (p == N.plim && e <= N.idlim);
}

struct RescanStats {
    int n_cand, n_kept;
    float max_kept;     // max over the set, plain max (no -1e30 floor)
    int first_kept;     // smallest id in the set
    int first_max_kept; // smallest id attaining max_kept
};

template <bool HAS_BIAS, bool HAS_ALLOW, class SM>
__device__ __forceinline__ RescanStats rescan_stats(const KArgs &A, SM &S, const float *row,
                                                    const uint32_t *abits, bool use_hash, float T,
                                                    bool use_ban, const Nucleus &N)
{
    int nc = 0, nk = 0, first = INT_MAX;
    float mk = -INFINITY;
    for (int e = threadIdx.x; e < A.V; e += WG) {
        const float yv = rescan_value<HAS_BIAS, HAS_ALLOW>(A, S, row, abits, use_hash, e);
        if (!(yv >= T)) continue;
        nc++;
        if (!in_nucleus(A, S, N, yv, e)) continue;
        if (use_ban && is_banned(S, e)) continue;
        nk++;
        mk = fmaxf(mk, yv);
        first = min(first, e);
    }
    RescanStats st;
    st.n_cand = block_sum(S, nc);
    st.n_kept = block_sum(S, nk);
    st.max_kept = block_max(S, mk);
    st.first_kept = block_min(S, first);
    int fm = INT_MAX;
    for (int e = threadIdx.x; e < A.V; e += WG) {
        const float yv = rescan_value<HAS_BIAS, HAS_ALLOW>(A, S, row, abits, use_hash, e);
        if (!(yv >= T) || !(yv == st.max_kept)) continue;
        if (!in_nucleus(A, S, N, yv, e)) continue;
        if (use_ban && is_banned(S, e)) continue;
        fm = min(fm, e);
    }
    st.first_max_kept = block_min(S, fm);
    return st;
}

// Sequential sum (draw == false) or draw (draw == true) over the row in id
// order, RS_CHUNK ids at a time.  Returns the sum; with draw, *token receives
// the first kept id whose running sum reaches r (-1 when none does).
template <bool HAS_BIAS, bool HAS_ALLOW, class SM>
__device__ __forceinline__ float rescan_sequential(const KArgs &A, SM &S, const float *row,
                                                   const uint32_t *abits, bool use_hash, float T,
                                                   bool use_ban, const Nucleus &N, float mx,
                                                   bool draw, float r, int *token)
{
    float *ep = S.u.ep + HSLOTS;  // histogram area; hval stays intact
    float acc = 0.0f;
    int found = -1;
    for (int c0 = 0; c0 < A.V; c0 += RS_CHUNK) {
        const int n = min(RS_CHUNK, A.V - c0);
        bool kept[RS_CHUNK / WG];
        __syncthreads();
#pragma unroll
        for (int q = 0; q < RS_CHUNK / WG; ++q) {
            const int i = (int)threadIdx.x + q * WG;
            kept[q] = false;
            if (i < n) {
                const int e = c0 + i;
                const float yv = rescan_value<HAS_BIAS, HAS_ALLOW>(A, S, row, abits, use_hash, e);
                kept[q] = (yv >= T) && in_nucleus(A, S, N, yv, e) && !(use_ban && is_banned(S, e));
                ep[i] = kept[q] ? glibc_expf((yv - mx) / A.T, S.exptab) : -1.0f;
            }
        }
        acc = block_seq_prefix(S, ep, n, acc);
        if (draw) {
            int first = INT_MAX;
#pragma unroll
            for (int q = 0; q < RS_CHUNK / WG; ++q) {
                const int i = (int)threadIdx.x + q * WG;
                if (i < n && kept[q] && r <= ep[i]) first = min(first, i);
            }
            first = block_min(S, first);
            if (first != INT_MAX) {
                found = c0 + first;
                break;
            }
        }
    }
    if (token) *token = found;
    return acc;
}

// Threshold of a row that holds nan values: the size-k min-heap of
// runtime/lal_sampling.h:69-104 (tools/server/qwen7b_server.c:238-256)
// replayed over the processed row in id order.  A nan never passes the heap's
// comparisons, so it rises to the root while the heap fills, sinks below
// values pushed after it and is never replaced; the root at the end is the
// threshold (nan when a nan is the root).  Wave 0 runs the replay: 16 chunks of
// 64 values are loaded at a time and staged in LDS; in a chunk, the first value
// that acts on the heap (any while it fills, then one above the root) is
// applied by lane 0, the root is re-read and the rest of the chunk filtered
// again.  The heap lives in S.cval and the staged values in S.cidx (the
// candidate buffers are not used on this path).
template <bool HAS_BIAS, bool HAS_ALLOW, class SM>
__device__ __forceinline__ float heap_replay_threshold(const KArgs &A, SM &S, const RowCtx &R, int k)
{
    constexpr int NB = 16;
    static_assert(sizeof(S.cidx) >= 64 * NB * sizeof(float), "staging area");
    float *hv = S.cval;
    float *stage = reinterpret_cast<float *>(S.cidx);
    __syncthreads();
    if (wave_id() == 0) {
        const int lane = lane_id();
        int size = 0;
        for (int base = 0; base < A.V; base += 64 * NB) {
            float xr[NB];
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int e = base + 64 * j + lane;
                xr[j] = (e < A.V) ? R.row[e] : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int e = base + 64 * j + lane;
                if (e < A.V)
                    stage[64 * j + lane] =
                        exact_value(R, e, upper_bound<HAS_BIAS, HAS_ALLOW>(A.bias, R.abits, e, xr[j]));
            }
            wave_sync();
            const int nch = min(NB, (A.V - base + 63) >> 6);
            for (int j = 0; j < nch; ++j) {
                const int c0 = base + 64 * j;
                const float x = (c0 + lane < A.V) ? stage[64 * j + lane] : 0.0f;
                unsigned long long todo = __ballot(c0 + lane < A.V);
                while (todo) {
                    const float root = hv[0];
                    const unsigned long long m = __ballot(size < k || x > root) & todo;
                    if (!m) break;
                    const int l = (int)__builtin_ctzll(m);
                    const float val = readlane_f(x, l);
                    if (lane == 0) {
                        if (size < k) {
                            int c = size;
                            hv[c] = val;
                            while (c > 0) {
                                const int p = (c - 1) >> 1;
                                if (hv[p] <= hv[c]) break;
                                const float t = hv[p];
                                hv[p] = hv[c];
                                hv[c] = t;
                                c = p;
                            }
                        } else {
                            hv[0] = val;
                            int p = 0;
                            for (;;) {
                                const int lc = 2 * p + 1, rc = 2 * p + 2;
                                int sm = p;
                                if (lc < size && hv[lc] < hv[sm]) sm = lc;
                                if (rc < size && hv[rc] < hv[sm]) sm = rc;
                                if (sm == p) break;
                                const float t = hv[p];
                                hv[p] = hv[sm];
                                hv[sm] = t;
                                p = sm;
                            }
                        }
                    }
                    if (size < k) ++size;
                    wave_sync();
                    todo &= (l == 63) ? 0ull : (~0ull << (l + 1));
                }
            }
            wave_sync();  // the staged chunk is read before the next one is written
        }
        if (lane == 0) S.redf[0] = hv[0];
    }
    __syncthreads();
    const float T = S.redf[0];
    __syncthreads();
    return T;
}

// Candidate outputs for a rescanned row: the first cand_ld pool ids in id
// order with their kept flag and probability e/sum.
template <bool HAS_BIAS, bool HAS_ALLOW, class SM>
__device__ __forceinline__ void rescan_write_cands(const KArgs &A, SM &S, const float *row,
                                                   const uint32_t *abits, bool use_hash, float T,
                                                   bool use_ban, const Nucleus &N, float mx, float sum,
                                                   bool greedy, int greedy_token, int b)
{
    constexpr int PT = RS_CHUNK / WG;
    int written = 0;
    for (int c0 = 0; c0 < A.V && written < A.cand_ld; c0 += RS_CHUNK) {
        const int n = min(RS_CHUNK, A.V - c0);
        int e_of[PT];
        float y_of[PT];
        int mine = 0;
#pragma unroll
        for (int q = 0; q < PT; ++q) {
            const int i = (int)threadIdx.x * PT + q;  // contiguous ids per thread
            e_of[q] = -1;
            y_of[q] = 0.0f;
            if (i < n) {
                const int e = c0 + i;
                y_of[q] = rescan_value<HAS_BIAS, HAS_ALLOW>(A, S, row, abits, use_hash, e);
                if (y_of[q] >= T) {
                    e_of[q] = e;
                    mine++;
                }
            }
        }
        int tot;
        int pos = written + block_excl_scan(mine, tot, S.wsum[(c0 / RS_CHUNK) & 1]);
#pragma unroll
        for (int q = 0; q < PT; ++q) {
            if (e_of[q] < 0) continue;
            if (pos < A.cand_ld) {
                const int e = e_of[q];
                const bool kept = greedy ? (e == greedy_token)
                                         : in_nucleus(A, S, N, y_of[q], e) && !(use_ban && is_banned(S, e));
                const size_t o = (size_t)b * A.cand_ld + pos;
                if (A.cand_ids) A.cand_ids[o] = e;
                if (A.cand_vals) A.cand_vals[o] = y_of[q];
                if (A.cand_kept) A.cand_kept[o] = kept ? 1 : 0;
                if (A.cand_probs)
                    A.cand_probs[o] = greedy ? (kept ? 1.0f : 0.0f)
                                             : (kept ? glibc_expf((y_of[q] - mx) / A.T, S.exptab) / sum : 0.0f);
            }
            pos++;
        }
        written += tot;
        __syncthreads();
    }
}

// The nucleus of a pool too large for the buffers.  All pool values are
// >= T and fewer than k exceed it, so the entries with p above p_T =
// p(T) (set A, fewer than k) are gathered and ranked in LDS; the rest share
// p == p_T and follow A in id order.  The cumulative mass is added
// sequentially in that order until it reaches top_p.
template <bool HAS_BIAS, bool HAS_ALLOW, class SM>
__device__ __forceinline__ Nucleus rescan_nucleus(const KArgs &A, SM &S, const float *row,
                                                  const uint32_t *abits, bool use_hash, float T,
                                                  int n_cand, float pool_max)
{
    Nucleus N;
    N.on = false;
    N.amax = (pool_max > -1e30f) ? pool_max : -1e30f;
    const float se = rescan_sequential<HAS_BIAS, HAS_ALLOW>(A, S, row, abits, use_hash, T, false, N,
                                                            N.amax, false, 0.0f, nullptr);
    N.inv = 1.0f / (se + 1e-12f);
    const float pT = glibc_expf((T - N.amax) / A.T, S.exptab) * N.inv;
    // gather A
    float *ap = S.cval;
    int *aid = S.cidx;
    float *sp = S.cval + LAL_GPU_MAX_K;
    int *sid = S.cidx + LAL_GPU_MAX_K;
    __syncthreads();
    if (threadIdx.x == 0) S.sel_rem = 0;
    __syncthreads();
    for (int e = threadIdx.x; e < A.V; e += WG) {
        const float yv = rescan_value<HAS_BIAS, HAS_ALLOW>(A, S, row, abits, use_hash, e);
        if (!(yv > T)) continue;
        const float p = glibc_expf((yv - N.amax) / A.T, S.exptab) * N.inv;
        if (!(p > pT)) continue;
        const int slot = atomicAdd(&S.sel_rem, 1);
        if (slot < LAL_GPU_MAX_K) {
            ap[slot] = p;
            aid[slot] = e;
        }
    }
    __syncthreads();
    const int na = min(S.sel_rem, LAL_GPU_MAX_K);
    // rank A by (p desc, id asc)
    for (int i = threadIdx.x; i < na; i += WG) {
        const float pi = ap[i];
        const int ii = aid[i];
        int rank = 0;
        for (int j = 0; j < na; ++j) {
            const float pj = ap[j];
            rank += (pj > pi) || (pj == pi && aid[j] < ii);
        }
        sp[rank] = pi;
        sid[rank] = ii;
    }
    __syncthreads();
    // cumulative mass in sorted order (one thread: the reference's order)
    if (threadIdx.x == 0) {
        float cum = 0.0f;
        int cut = -1;
        for (int i = 0; i < na; ++i) {
            cum = cum + sp[i];
            if (cum >= A.top_p) {
                cut = i;
                break;
            }
        }
        int jg = 0;  // tokens of the tie group kept (0: cut inside A; n_g: all)
        const int ng = n_cand - na;
        if (cut < 0) {
            jg = ng;
            for (int j = 1; j <= ng; ++j) {
                cum = cum + pT;
                if (cum >= A.top_p) {
                    jg = j;
                    break;
                }
            }
        }
        S.redf[0] = (cut >= 0) ? sp[cut] : pT;
        S.redi[0] = (cut >= 0) ? sid[cut] : -1;
        S.redi2[0] = (cut >= 0) ? 0 : jg;
    }
    __syncthreads();
    N.on = true;
    N.plim = S.redf[0];
    N.idlim = S.redi[0];
    const int jg = S.redi2[0];
    __syncthreads();
    if (N.idlim < 0) {
        // the cut falls in the tie group: the id of its jg-th member (id order)
        constexpr int PT = RS_CHUNK / WG;
        int seen = 0, found = A.V;
        for (int c0 = 0; c0 < A.V && jg > 0; c0 += RS_CHUNK) {
            const int n = min(RS_CHUNK, A.V - c0);
            int mine = 0;
            bool g[PT];
#pragma unroll
            for (int q = 0; q < PT; ++q) {
                const int i = (int)threadIdx.x * PT + q;  // contiguous ids per thread
                g[q] = false;
                if (i < n) {
                    const int e = c0 + i;
                    const float yv = rescan_value<HAS_BIAS, HAS_ALLOW>(A, S, row, abits, use_hash, e);
                    if (yv >= T) {
                        const float p = glibc_expf((yv - N.amax) / A.T, S.exptab) * N.inv;
                        g[q] = (p == pT);
                    }
                    mine += g[q];
                }
            }
            int tot;
            int pos = seen + block_excl_scan(mine, tot, S.wsum[(c0 / RS_CHUNK) & 1]);
            int hit = INT_MAX;
#pragma unroll
            for (int q = 0; q < PT; ++q) {
                if (!g[q]) continue;
                pos++;
                if (pos == jg) hit = c0 + (int)threadIdx.x * PT + q;
            }
            hit = block_min(S, hit);
            seen += tot;
            if (hit != INT_MAX) {
                found = hit;
                break;
            }
        }
        N.idlim = found;
        N.plim = pT;
    }
    return N;
}

// ---------------------------------------------------------------------------
// Epilogue over the pool (ids ascending in S.cidx[0..nc), values in S.cval)
// when it fits one wave: one candidate per lane of wave 0, no barriers.
// ---------------------------------------------------------------------------
struct RowResult {
    int token, n_kept;
    float sum;
};

// Sequential fp32 helpers over one wave's 64 values staged in LDS (buf,
// 64 floats): every lane runs the same addition chain in index order, which is
// the reference's scalar loop order.  Values that are not in the set must be
// +0.0 (adding +0.0 to a sum of non-negative terms leaves it unchanged).
struct Staged64 {
    f32x4 q[16];
};

__device__ __forceinline__ Staged64 load_staged(const float *buf)
{
    Staged64 s;
#pragma unroll
    for (int i = 0; i < 16; ++i) s.q[i] = reinterpret_cast<const f32x4 *>(buf)[i];
    return s;
}

// Sum of the staged values [0, n) in index order.  Entries from n to 63 are
// +0.0, so the sum stops after the quad holding entry n - 1 (n is uniform).
__device__ __forceinline__ float seq_total(const float *buf, int n)
{
    const Staged64 s = load_staged(buf);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if (4 * i < n) {
            acc = acc + s.q[i][0];
            acc = acc + s.q[i][1];
            acc = acc + s.q[i][2];
            acc = acc + s.q[i][3];
        }
    }
    return acc;
}

// First index i < n whose inclusive sequential prefix reaches `target`
// (prefix >= target); n if none.  The prefix never decreases (non-negative
// terms), so the index is the number of prefixes that do not reach target,
// clamped to n; prefixes past the quad holding entry n - 1 cannot change it.
__device__ __forceinline__ int seq_first_reach(const float *buf, int n, float target)
{
    const Staged64 s = load_staged(buf);
    float acc = 0.0f;
    int below = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if (4 * i < n) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                acc = acc + s.q[i][c];
                below += !(acc >= target) ? 1 : 0;  // a nan target is never reached
            }
        }
    }
    return min(below, n);
}

// Pool of at most 64 candidates, one per lane in ascending id order (S.cval /
// S.cidx [0, nc)), handled by one wave.
template <class SM>
__device__ __forceinline__ RowResult wave_epilogue(const KArgs &A, SM &S, int nc, float u, int b)
{
    const int lane = lane_id();
    const bool valid = lane < nc;
    const float y = valid ? S.cval[lane] : -INFINITY;
    const int id = valid ? S.cidx[lane] : -1;
    const bool ban = valid && A.any_bans && is_banned(S, id);
    float *buf = S.u.ep;          // 64 staged values
    float *buf2 = S.u.ep + 64;    // sorted probabilities
    bool nuc = valid;
    float amax = -1e30f, e1 = 0.0f;
    const bool top_p_on = A.top_p > 0.0f && A.top_p < 1.0f;
    if (top_p_on) {
        // gpt2_server.c:2908-2955: probabilities over the pool, stable sort
        // by descending probability, inclusive cumulative cutoff
        amax = wave_max(valid ? y : -INFINITY);
        if (!(amax > -1e30f)) amax = -1e30f;
        e1 = valid ? glibc_expf((y - amax) / A.T, S.exptab) : 0.0f;
        buf[lane] = e1;
        wave_sync();
        const float se = seq_total(buf, nc);
        const float inv = 1.0f / (se + 1e-12f);
        const float p = valid ? e1 * inv : -1.0f;
        // rank in (probability desc, id asc) order: 64-bit keys, larger first
        const uint64_t key = valid ? (((uint64_t)fkey(p) << 32) | (uint32_t)(63 - lane)) : 0ull;
        uint64_t *kb = reinterpret_cast<uint64_t *>(S.u.ep + 128);
        kb[lane] = key;  // 0 past the pool: below every valid key
        wave_sync();
        int rank = 0;
        for (int j = 0; j < nc; j += 2) {  // key 0 at nc (odd nc): below every valid key
            const ulonglong2 kk = reinterpret_cast<const ulonglong2 *>(kb)[j >> 1];
            rank += (kk.x > key) + (kk.y > key);
        }
        buf2[lane] = 0.0f;
        wave_sync();
        if (valid) buf2[rank] = p;
        wave_sync();
        const int cut = min(seq_first_reach(buf2, nc, A.top_p), nc - 1);
        nuc = valid && rank <= cut;
        wave_sync();
    }
    bool kept = nuc && !ban;
    if (__ballot(kept) == 0ull) kept = valid;  // restore the top-k pool
    const int n_kept = __popcll(__ballot(kept));
    const float kmax = wave_max(kept ? y : -INFINITY);
    const float mx = (kmax > -1e30f) ? kmax : -1e30f;
    // same inputs as e1 when the maximum is kept: reuse it
    const float e2 = !kept ? 0.0f : (top_p_on && mx == amax) ? e1 : glibc_expf((y - mx) / A.T, S.exptab);
    buf[lane] = e2;
    wave_sync();
    const float sum = seq_total(buf, nc);
    RowResult res;
    res.n_kept = n_kept;
    res.sum = sum;
    if (A.variant == LAL_GPU_VARIANT_FILTERED && sum <= 0.0f) {
        const unsigned long long hm = __ballot(kept && y == kmax && kmax > -1e30f);
        res.token = hm ? readlane_i(id, (int)__builtin_ctzll(hm)) : 0;
    } else {
        const float r = u * sum;
        if ((A.flags & LAL_GPU_F_DRAW_GPT2) && r == 0.0f) {
            res.token = 0;
        } else {
            // first kept candidate (id order) whose prefix reaches r.  A
            // non-kept entry carries its predecessor's prefix, so for r > 0 the
            // first index found is kept; for r <= 0 it is the first kept one.
            int f;
            if (r <= 0.0f) {
                const unsigned long long hk = __ballot(kept);
                f = hk ? (int)__builtin_ctzll(hk) : nc;
            } else {
                f = seq_first_reach(buf, nc, r);
            }
            res.token = (f < nc) ? readlane_i(id, f) : A.fallback;
        }
    }
    if (valid && lane < A.cand_ld) {
        const size_t o = (size_t)b * A.cand_ld + lane;
        if (A.cand_ids) A.cand_ids[o] = id;
        if (A.cand_vals) A.cand_vals[o] = y;
        if (A.cand_kept) A.cand_kept[o] = kept ? 1 : 0;
        if (A.cand_probs) A.cand_probs[o] = kept ? e2 / sum : 0.0f;
    }
    wave_sync();
    return res;
}

// General epilogue (pool above one wave): block-wide, PER entries per thread.
template <int PER, class SM>
__device__ __forceinline__ RowResult block_epilogue(const KArgs &A, SM &S, int nc, float u, int b)
{
    const int tid = threadIdx.x;
    float *ep = S.u.ep;
    float yv[PER];
    bool nuc[PER], ban[PER], kept[PER];
#pragma unroll
    for (int r = 0; r < PER; ++r) {
        const int j = tid + r * WG;
        yv[r] = (j < nc) ? S.cval[j] : NAN;
        nuc[r] = (j < nc);
        ban[r] = (j < nc) && A.any_bans && is_banned(S, S.cidx[j]);
    }
    if (A.top_p > 0.0f && A.top_p < 1.0f) {
        float lm = -INFINITY;
#pragma unroll
        for (int r = 0; r < PER; ++r)
            if (tid + r * WG < nc) lm = fmaxf(lm, yv[r]);
        float amax = block_max(S, lm);
        if (!(amax > -1e30f)) amax = -1e30f;
        float e1[PER];
#pragma unroll
        for (int r = 0; r < PER; ++r) {
            const int j = tid + r * WG;
            e1[r] = (j < nc) ? glibc_expf((yv[r] - amax) / A.T, S.exptab) : 0.0f;
            if (j < nc) ep[j] = e1[r];
        }
        const float se = block_seq_prefix(S, ep, nc, 0.0f);
        const float inv = 1.0f / (se + 1e-12f);
        float pr[PER];
#pragma unroll
        for (int r = 0; r < PER; ++r) {
            const int j = tid + r * WG;
            pr[r] = e1[r] * inv;
            if (j < nc) ep[j] = pr[r];
        }
        __syncthreads();
        int prk[PER];
#pragma unroll
        for (int r = 0; r < PER; ++r) {
            const int j = tid + r * WG;
            prk[r] = -1;
            if (j < nc) {
                int rank = 0, q = 0;
                for (; q + 8 <= nc; q += 8) {  // eight LDS reads in flight
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const float pq = ep[q + u];
                        rank += (pq > pr[r]) || (pq == pr[r] && q + u < j);
                    }
                }
                for (; q < nc; ++q) {
                    const float pq = ep[q];
                    rank += (pq > pr[r]) || (pq == pr[r] && q < j);
                }
                prk[r] = rank;
            }
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < PER; ++r)
            if (prk[r] >= 0) ep[prk[r]] = pr[r];
        block_seq_prefix(S, ep, nc, 0.0f);
        int fc = INT_MAX;
#pragma unroll
        for (int r = 0; r < PER; ++r) {
            const int j = tid + r * WG;
            if (j < nc && ep[j] >= A.top_p) fc = min(fc, j);
        }
        fc = block_min(S, fc);
        const int cut = (fc == INT_MAX) ? nc - 1 : fc;
#pragma unroll
        for (int r = 0; r < PER; ++r) nuc[r] = (prk[r] >= 0) && (prk[r] <= cut);
    }
    int lk = 0;
#pragma unroll
    for (int r = 0; r < PER; ++r) {
        kept[r] = nuc[r] && !ban[r];
        lk += kept[r];
    }
    RowResult res;
    res.n_kept = block_sum(S, lk);
    if (res.n_kept == 0) {
#pragma unroll
        for (int r = 0; r < PER; ++r) kept[r] = (tid + r * WG < nc);
        res.n_kept = nc;
    }
    float lm = -INFINITY;
#pragma unroll
    for (int r = 0; r < PER; ++r)
        if (kept[r]) lm = fmaxf(lm, yv[r]);
    const float kmax = block_max(S, lm);
    const float mx = (kmax > -1e30f) ? kmax : -1e30f;
    float e2[PER];
#pragma unroll
    for (int r = 0; r < PER; ++r) {
        const int j = tid + r * WG;
        e2[r] = kept[r] ? glibc_expf((yv[r] - mx) / A.T, S.exptab) : 0.0f;
        if (j < nc) ep[j] = kept[r] ? e2[r] : -1.0f;
    }
    res.sum = block_seq_prefix(S, ep, nc, 0.0f);
    if (A.variant == LAL_GPU_VARIANT_FILTERED && res.sum <= 0.0f) {
        int cand = INT_MAX;
#pragma unroll
        for (int r = 0; r < PER; ++r)
            if (kept[r] && yv[r] == kmax && kmax > -1e30f) cand = min(cand, tid + r * WG);
        const int j = block_min(S, cand);
        res.token = (j == INT_MAX) ? 0 : S.cidx[j];
    } else {
        const float rr = u * res.sum;
        if ((A.flags & LAL_GPU_F_DRAW_GPT2) && rr == 0.0f) {
            res.token = 0;
        } else {
            int cand = INT_MAX;
#pragma unroll
            for (int r = 0; r < PER; ++r)
                if (kept[r] && rr <= ep[tid + r * WG]) cand = min(cand, tid + r * WG);
            const int j = block_min(S, cand);
            res.token = (j == INT_MAX) ? A.fallback : S.cidx[j];
        }
    }
    if (A.cand_ld > 0) {
#pragma unroll
        for (int r = 0; r < PER; ++r) {
            const int j = tid + r * WG;
            if (j < nc && j < A.cand_ld) {
                const size_t o = (size_t)b * A.cand_ld + j;
                if (A.cand_ids) A.cand_ids[o] = S.cidx[j];
                if (A.cand_vals) A.cand_vals[o] = S.cval[j];
                if (A.cand_kept) A.cand_kept[o] = kept[r] ? 1 : 0;
                if (A.cand_probs) A.cand_probs[o] = kept[r] ? e2[r] / res.sum : 0.0f;
            }
        }
    }
    return res;
}

// ---------------------------------------------------------------------------
// The sampler kernel: one workgroup (four wave64) per row.
// ---------------------------------------------------------------------------
// LIST: list mode (an LM head's candidate lists), at most 16 rows of one
// workgroup each, so no occupancy target
template <bool HAS_BIAS, bool HAS_ALLOW, int CAPW, bool LIST = false>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(LIST ? 1 : 4, 8))) void sample_rows_kernel(KArgs A)
{
    __shared__ Smem<CAPW> S;
    constexpr int PER = NWAVE * CAPW / WG;  // union entries per thread
    // work unit: slice `sl` of row `b`.  Rows go in groups of 8 with the
    // slices of one row 8 workgroups apart, so that (with workgroups dealt
    // round-robin to the 8 XCDs) every slice of a row runs on the same XCD
    // and its list exchange stays in that XCD's L2.
    const int nsl = A.nslice;
    int b, sl;
    {
        const int per_grp = 8 * nsl;
        const int gi = blockIdx.x / per_grp;
        const int r = blockIdx.x - gi * per_grp;
        sl = r >> 3;
        b = gi * 8 + (r & 7);
    }
    if (b >= A.batch) return;
    // The vector memory issue arbitration of a CU prefers older waves, so the
    // four workgroups resident on a CU stream at different rates.  One
    // priority step for the youngest (grid index in [3 ncu, 4 ncu)) sets the
    // fastest end for one workgroup per row; with sliced rows (prio_rotate)
    // the priority rotates over the four every four stream iterations
    // instead, so that every slice of a row gets each rank in turn.
    const int pslot = ((int)blockIdx.x / A.ncu) & 3;
    if (!A.prio_rotate && pslot == 3) __builtin_amdgcn_s_setprio(1);
    const int tid = threadIdx.x;
    const int w = wave_id(), lane = lane_id();
    const int V = A.V;
    const float *row = A.logits + (size_t)b * A.ld;
    const uint32_t *abits = HAS_ALLOW ? A.allow + (size_t)b * A.allow_ld : nullptr;
    const int *hrow = A.hist ? A.hist + (size_t)b * A.hist_ld : nullptr;
    int nh = 0;
    if (hrow) {
        nh = A.hist_len ? A.hist_len[b] : A.hist_ld;
        nh = max(0, min(nh, A.hist_ld));
    }
    // history / ban ids first: the setup waits for these loads only
    // (LAL_GPU_MAX_HISTORY is two per thread)
    static_assert(LAL_GPU_MAX_HISTORY <= 2 * WG && LAL_GPU_MAX_BAN_IDS <= WG, "setup registers");
    const int h0 = (tid < nh) ? hrow[tid] : -1;
    const int h1 = (tid + WG < nh) ? hrow[tid + WG] : -1;
    const int bid = (tid < A.n_ban) ? A.ban_ids[tid] : -1;
    const int last_tok = (A.last_tokens && A.ban_last) ? A.last_tokens[b] : -1;
    const uint64_t xtab = (tid < 32) ? kExp2Tab[tid] : 0ull;
    const uint32_t bpk = (HAS_BIAS && tid < A.bias_nparts) ? A.bias_part[tid] : 0u;
    // list mode: the row's candidates are complete when the list holds at
    // least k values above the largest bound the head filtered with (checked
    // after the list pass); a full list, a nan logit or no bound: the row is
    // streamed
    int hcnt = 0;
    int hsc[HSUB];  // entries of each sub-list
    uint32_t hkey = 0u;
    bool list_ok = false;
    if (LIST) {
        const int4 hm = A.hmeta[(size_t)b * HMETA_STRIDE];
        list_ok = (hm.w & 3) == 0;
#pragma unroll
        for (int q = 0; q < HSUB; ++q) {
            hsc[q] = A.hmeta[(size_t)b * HMETA_STRIDE + 1 + q].x;
            list_ok = list_ok && hsc[q] >= 0 && hsc[q] <= A.hcap / HSUB;
            hcnt += hsc[q];
        }
    }

    const RowGeo g = row_geo(row, V);
    const int k = A.greedy ? 1 : min(max(A.k, 1), V);

    // this slice's quads of the aligned body, and this wave's contiguous share
    const int sb = (int)(((long long)g.nb4 * sl) / nsl);
    const int se = (int)(((long long)g.nb4 * (sl + 1)) / nsl);
    const int qb = sb + (int)(((long long)(se - sb) * w) / NWAVE);
    const int qe = sb + (int)(((long long)(se - sb) * (w + 1)) / NWAVE);
    const bool has_extras = (sl == 0) && (g.head + g.ntail > 0);
    const int vlen = 4 * (se - sb) + (has_extras ? g.head + g.ntail : 0);
    const f32x4 *row4 = reinterpret_cast<const f32x4 *>(row + g.head);
    // allow and bias-nonzero bits: lane l holds word l of the 34 words under
    // a wave-iteration (the window starts at the word of its first element)
    const int nwords = (V + 31) >> 5;
    auto wload = [&](const uint32_t *bits, int q) -> uint32_t {
        const int wi = ((g.head + 4 * q) >> 5) + lane;
        return (lane < 34 && wi < nwords) ? bits[wi] : 0u;
    };
    uint32_t aw0 = 0u, aw1 = 0u, bw0 = 0u, bw1 = 0u;

    f32x4 cur[U4], nx1[U4];
    // few workgroups (a small batch): the first two stream iterations go out
    // with the sample, nothing queues behind them
    const bool early = A.batch <= 16;
    if (early && !LIST) {
#pragma unroll
        for (int u = 0; u < U4; ++u) {
            const int q = qb + u * 64 + lane;
            cur[u] = (q < qe) ? __builtin_nontemporal_load(row4 + q) : f32x4{NAN, NAN, NAN, NAN};
            const int q1 = qb + WITER + u * 64 + lane;
            nx1[u] = (q1 < qe) ? __builtin_nontemporal_load(row4 + q1) : f32x4{NAN, NAN, NAN, NAN};
        }
        if (HAS_ALLOW) {
            aw0 = wload(abits, qb);
            aw1 = wload(abits, qb + WITER);
        }
        if (HAS_BIAS) {
            bw0 = wload(A.bias_bits, qb);
            bw1 = wload(A.bias_bits, qb + WITER);
        }
    }
    // the slice sample goes out first, alone: every workgroup waits for its
    // sample, and stream loads queued with it would only delay it
    f32x4 smp[SR];
#pragma unroll
    for (int r = 0; r < SR; ++r) {
        const int sidx = tid + WG * r;
        const int q = sb + (sidx >> 6) * SBLK + (sidx & 63);
        smp[r] = (q < se && !LIST) ? row4[q] : f32x4{NAN, NAN, NAN, NAN};
    }

    // ---- setup: hash of history / ban ids, and the threshold estimate ----
    // tau_est = the ks-th largest of the per-thread maxima of the sampled
    // upper bounds (a subset of the sample, so no larger than the sample's
    // ks-th largest); ks is chosen so that with the sampling fraction f the
    // sample holds fewer than ks of the row's top-k except with negligible
    // probability.  It is verified after streaming (>= k captured values) and
    // the row is streamed again without it when the check fails.
    unsigned *skeys = S.u.h.whist[0];  // 4 x 64 sample keys
    int nsmp = 0;                      // sampled positions (closed form)
    for (int jb = 0; jb < SR * NWAVE; ++jb) {
        const int st0 = sb + jb * SBLK;
        if (st0 < se) nsmp += 4 * min(64, se - st0);
    }
    const float lam = (float)k * (float)nsmp / (float)max(vlen, 1);
    const int ks = (int)ceilf(lam + 6.0f * sqrtf(lam) + 6.0f);
    const bool use_est = !LIST && !A.greedy && nsmp > 0 && ks <= 64;
    {
        float lm = -INFINITY;
#pragma unroll
        for (int r = 0; r < SR; ++r) {
            const int sidx = tid + WG * r;
            const int q = sb + (sidx >> 6) * SBLK + (sidx & 63);
            if (q < se) {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    lm = fmaxf(lm, upper_bound<HAS_BIAS, HAS_ALLOW>(A.bias, abits, g.head + 4 * q + c,
                                                                   smp[r][c]));
            }
        }
        skeys[tid] = (lm == lm && lm > -INFINITY) ? fkey(lm) : 0u;
    }
    // the first two iterations' loads fly during the hash setup and estimate
    if (!early && !LIST) {
#pragma unroll
        for (int u = 0; u < U4; ++u) {
            const int q = qb + u * 64 + lane;
            cur[u] = (q < qe) ? __builtin_nontemporal_load(row4 + q) : f32x4{NAN, NAN, NAN, NAN};
            const int q1 = qb + WITER + u * 64 + lane;
            nx1[u] = (q1 < qe) ? __builtin_nontemporal_load(row4 + q1) : f32x4{NAN, NAN, NAN, NAN};
        }
        if (HAS_ALLOW) {
            aw0 = wload(abits, qb);
            aw1 = wload(abits, qb + WITER);
        }
        if (HAS_BIAS) {
            bw0 = wload(A.bias_bits, qb);
            bw1 = wload(A.bias_bits, qb + WITER);
        }
    }
    for (int s = tid; s < HSLOTS; s += WG) {
        S.hkey[s] = -1;
        S.hinfo[s] = 0;
    }
    if (tid < 32) S.exptab[tid] = xtab;
    if (tid == 0) {
        S.nan_flag = 0;
        S.bias_key = 0u;
    }
    __syncthreads();
    if (HAS_BIAS) {
        const uint32_t m = wave_max_u(bpk);
        if (lane == 0) atomicMax(&S.bias_key, m);
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int i = tid + r * WG;
        const int t = r ? h1 : h0;
        if (i >= nh || t < 0 || t >= V) continue;
        int flags = 0;
        if (A.mask_recent > 0 && i >= nh - A.mask_recent) flags |= HF_MASKPRE;
        if (A.ban_last && !A.last_tokens && i == nh - 1) flags |= HF_BAN;
        if (A.ban_repeat > 0 && i >= nh - A.ban_repeat) flags |= HF_BAN;
        hash_insert(S.hkey, S.hinfo, t, A.apply_pen ? 1 : 0, flags);
    }
    if (bid >= 0 && bid < V) hash_insert(S.hkey, S.hinfo, bid, 0, HF_BAN);
    if (tid == 0 && last_tok >= 0 && last_tok < V) hash_insert(S.hkey, S.hinfo, last_tok, 0, HF_BAN);
    if (use_est && w == 0) {
        // the ks-th largest of the 256 keys, bit by bit (ballot counts)
        const uint32_t k0 = skeys[lane], k1 = skeys[64 + lane], k2 = skeys[128 + lane],
                       k3 = skeys[192 + lane];
        uint32_t K = 0u;
        for (int bit = 31; bit >= 0; --bit) {
            const uint32_t cand = K | (1u << bit);
            const int c = __popcll(__ballot(k0 >= cand)) + __popcll(__ballot(k1 >= cand)) +
                          __popcll(__ballot(k2 >= cand)) + __popcll(__ballot(k3 >= cand));
            if (c >= ks) K = cand;
        }
        if (lane == 0) S.sel_rem = (int)K;
    }
    __syncthreads();
    float tau_est = -INFINITY;
    if (use_est) {
        const uint32_t kk = (uint32_t)S.sel_rem;
        if (kk) tau_est = keyf(kk);
    }
    if (LIST) {
        // the head's bound from the final slots (at least every bound a wave
        // filtered with, so the list holds every value at or above it)
        if (w == 0) {
            const uint32_t K = wave_kth_lane_key(A.hslots[(size_t)b * 64 + lane], A.hks);
            if (lane == 0) S.sel_rem = (int)K;
        }
        __syncthreads();
        hkey = (uint32_t)S.sel_rem;
        __syncthreads();
        if (hkey == 0u) list_ok = false;
        if (list_ok) tau_est = keyf(hkey);
    }
    // bound of bias[e] for a set bias bit (a nan when one flagged entry is a
    // nan or -inf: those rows take the nan path, which reads the bias itself)
    const float bmax = HAS_BIAS ? keyf(S.bias_key) : 0.0f;
    const bool use_hash = (nh > 0) || (A.n_ban > 0);
    RowCtx R;
    R.row = row;
    R.bias = A.bias;
    R.abits = abits;
    R.hkey = S.hkey;
    R.hinfo = S.hinfo;
    R.pen = A.pen;
    R.has_bias = HAS_BIAS;
    R.has_allow = HAS_ALLOW;
    R.use_hash = use_hash;
    R.bound_bias = HAS_BIAS;
    R.bias_bits = A.bias_bits;

    float *bv = S.cval + w * CAPW;
    int *bi = S.cidx + w * CAPW;
    unsigned *hist = S.u.h.whist[w];
    // a lane's 4 bits of a window can straddle two words unless the row's
    // aligned body starts on a multiple of 4 elements
    const bool two_words = g.head != 0;
    WState st;
    for (int attempt = 0; attempt < 2; ++attempt) {
        // list mode: the first pass reads the head's list, not the row
        const bool from_list = LIST && list_ok && attempt == 0;
        if (attempt == 1 || (LIST && !list_ok)) {
            // the estimate was above the row's k-th largest: stream again.  The
            // share's start goes through an opaque copy, so that the compiler
            // recomputes these loads' masks and addresses here instead of
            // holding the first pass's across the whole stream.
            int qa = __builtin_amdgcn_readfirstlane(qb);
            asm volatile("" : "+s"(qa));
#pragma unroll
            for (int u = 0; u < U4; ++u) {
                const int q = qa + u * 64 + lane;
                cur[u] = (q < qe) ? __builtin_nontemporal_load(row4 + q) : f32x4{NAN, NAN, NAN, NAN};
                const int q1 = qa + WITER + u * 64 + lane;
                nx1[u] = (q1 < qe) ? __builtin_nontemporal_load(row4 + q1) : f32x4{NAN, NAN, NAN, NAN};
            }
            if (HAS_ALLOW) {
                aw0 = wload(abits, qa);
                aw1 = wload(abits, qa + WITER);
            }
            if (HAS_BIAS) {
                bw0 = wload(A.bias_bits, qa);
                bw1 = wload(A.bias_bits, qa + WITER);
            }
        }
        __syncthreads();
        if (tid == 0) S.tau_key = (tau_est > -INFINITY) ? fkey(tau_est) : 0u;
        __syncthreads();
        st.tau = -INFINITY;
        st.strict = 0;
        st.cnt = 0;
        st.tcmp = -INFINITY;

    if (from_list) {
        // every list value is a raw logit of an id the head computed once;
        // the waves take 64 entries of the sub-lists' concatenation at a
        // time, in rotation
        const float *lv = A.lst_val + (size_t)b * A.hcap;
        const int *li = A.lst_idx + (size_t)b * A.hcap;
        const int subcap = A.hcap / HSUB;
        for (int j0 = w * 64; j0 < hcnt; j0 += NWAVE * 64) {
            const int j = j0 + lane;
            int sq = 0, off = j;  // entry j: sub-list sq, entry off
#pragma unroll
            for (int q = 0; q < HSUB - 1; ++q)
                if (sq == q && off >= hsc[q]) {
                    off -= hsc[q];
                    sq = q + 1;
                }
            float x[4] = {NAN, NAN, NAN, NAN};
            int eb[1] = {0};
            if (j < hcnt) {
                x[0] = lv[sq * subcap + off];
                eb[0] = li[sq * subcap + off];
            }
            const float tsh = keyf(S.tau_key);
            const float tcmp = (st.tcmp != st.tcmp) ? st.tcmp : fmaxf(st.tcmp, tsh);
            unsigned long long pm[4] = {__ballot(x[0] >= tcmp), 0ull, 0ull, 0ull};
            if (pm[0]) wave_offer<1, CAPW>(bv, bi, hist, R, x, pm, eb, tcmp, st, k, &S.tau_key);
        }
    } else {
    // ---- stream: each wave owns its share, no workgroup barrier ----------
    if (w == 0 && has_extras) {
        // head / tail elements outside the aligned body (slice 0)
        const int e = extra_elem(g, lane);
        float x[4] = {NAN, NAN, NAN, NAN};
        const int eb[1] = {e};
        if (e >= 0) x[0] = upper_bound<HAS_BIAS, HAS_ALLOW>(A.bias, abits, e, row[e]);
        if (__ballot(e >= 0 && x[0] != x[0]) && lane == 0) S.nan_flag = 1;
        unsigned long long pm[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) pm[i] = __ballot(x[i] >= -INFINITY);
        wave_offer<1, CAPW>(bv, bi, hist, R, x, pm, eb, -INFINITY, st, k, &S.tau_key);
    }
    // One wave-iteration: filter the values `c` of quads [q0, q0 + WITER)
    // (allow / bias words awc, bwc) and issue the loads of the iteration two
    // ahead into `n2` (words into awn, bwn), every load at a clamped address
    // (lanes past the share are set to nan where the values are used).  For
    // the large-k instantiation the three register sets rotate by unrolling
    // the loop three times, never by copies: a copy of a register still
    // being loaded waits for that load, which drained every load in flight
    // once per iteration.
    auto iter = [&](int q0, const f32x4 (&c)[U4], f32x4 (&n2)[U4], uint32_t awc, uint32_t bwc, uint32_t &awn,
                    uint32_t &bwn) __attribute__((always_inline)) {
        if (A.prio_rotate) {
            const int itn = (q0 - qb) / WITER;
            if ((itn & 3) == 0) {
                switch ((pslot + (itn >> 2)) & 3) {
                case 0: __builtin_amdgcn_s_setprio(0); break;
                case 1: __builtin_amdgcn_s_setprio(1); break;
                case 2: __builtin_amdgcn_s_setprio(2); break;
                default: __builtin_amdgcn_s_setprio(3); break;
                }
            }
        }
        awn = HAS_ALLOW ? wload(abits, q0 + 2 * WITER) : 0u;
        bwn = HAS_BIAS ? wload(A.bias_bits, q0 + 2 * WITER) : 0u;
#pragma unroll
        for (int u = 0; u < U4; ++u)
            n2[u] = __builtin_nontemporal_load(row4 + min(q0 + 2 * WITER + u * 64 + lane, qe - 1));
        // effective filter: own threshold, or the largest any wave of this
        // row has reached (each is a lower bound of the row's k-th largest);
        // a strict threshold becomes ">=" against the next float up
        // (keyf(0), "none", is a nan and drops out of the fmaxf; a nan own
        // filter passes nothing and stays)
        const float tsh = keyf(S.tau_key);
        const float tcmp = (st.tcmp != st.tcmp) ? st.tcmp : fmaxf(st.tcmp, tsh);
        // processed-value upper bounds (values of invalid lanes are nan)
        // (a set bias bit adds the bias maximum: an upper bound, resolved
        // from bias[e] when the entry is refined; a clear one adds +0.0, which
        // is bias[e] itself)
        float x[VPL];
#pragma unroll
        for (int u = 0; u < U4; ++u) {
            const int rel = ((g.head + 4 * q0) & 31) + 256 * u + 4 * lane;
            const uint32_t ab = HAS_ALLOW ? window_nibble(awc, rel, two_words) : 0xFu;
            const uint32_t bb = HAS_BIAS ? window_nibble(bwc, rel, two_words) : 0u;
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                float v = c[u][cc];
                if (HAS_BIAS) v = v + (((bb >> cc) & 1u) ? bmax : 0.0f);
                if (HAS_ALLOW && !((ab >> cc) & 1u)) v = -INFINITY;
                x[4 * u + cc] = v;
            }
        }
        if (q0 + WITER > qe) {
            // partial last iteration: lanes past the share (loaded at a
            // clamped address) stay out
#pragma unroll
            for (int u = 0; u < U4; ++u)
                if (q0 + u * 64 + lane >= qe)
#pragma unroll
                    for (int cc = 0; cc < 4; ++cc) x[4 * u + cc] = NAN;
        }
        // a nan never passes the filter; the row's nans are found here, two
        // values per unordered compare (padding lanes of a partial
        // iteration are nan too and stay out)
        {
            unsigned long long nanm = 0ull;
#pragma unroll
            for (int u = 0; u < U4; ++u) {
                unsigned long long nu = __ballot(__builtin_isunordered(x[4 * u], x[4 * u + 1])) |
                                        __ballot(__builtin_isunordered(x[4 * u + 2], x[4 * u + 3]));
                if (q0 + WITER > qe) nu &= __ballot(q0 + u * 64 + lane < qe);
                nanm |= nu;
            }
            if (nanm && lane == 0) S.nan_flag = 1;
        }
        unsigned long long pm[VPL], any = 0ull;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            pm[i] = __ballot(x[i] >= tcmp);
            any |= pm[i];
        }
        if (any) {
            int eb[U4];
#pragma unroll
            for (int u = 0; u < U4; ++u) eb[u] = g.head + 4 * (q0 + u * 64 + lane);
            wave_offer<U4, CAPW>(bv, bi, hist, R, x, pm, eb, tcmp, st, k, &S.tau_key);
        }
    };
    if constexpr (CAPW > CAPW_SMALL) {
        f32x4 nx2[U4];
        uint32_t aw2 = 0u, bw2 = 0u;
        for (int q0 = qb; q0 < qe; q0 += 3 * WITER) {
            iter(q0, cur, nx2, aw0, bw0, aw2, bw2);
            if (q0 + WITER >= qe) break;
            iter(q0 + WITER, nx1, cur, aw1, bw1, aw0, bw0);
            if (q0 + 2 * WITER >= qe) break;
            iter(q0 + 2 * WITER, nx2, nx1, aw2, bw2, aw1, bw1);
        }
    } else {
        // within the 128 registers of four workgroups per CU the third set
        // does not fit: the sets rotate by copies (the loads of the
        // iteration two ahead fly while this one is filtered)
        for (int q0 = qb; q0 < qe; q0 += WITER) {
            f32x4 nx2[U4];
            uint32_t aw2 = 0u, bw2 = 0u;
            iter(q0, cur, nx2, aw0, bw0, aw2, bw2);
#pragma unroll
            for (int u = 0; u < U4; ++u) {
                cur[u] = nx1[u];
                nx1[u] = nx2[u];
            }
            aw0 = aw1;
            aw1 = aw2;
            bw0 = bw1;
            bw1 = bw2;
        }
    }
    }  // stream
    // resolve the entries still holding upper bounds (below the estimate:
    // dropped, so the count below verifies it)
    if (use_hash || HAS_BIAS) wave_refine_batched(bv, bi, st.cnt, R, tau_est, false);
    int alive = 0;
    uint32_t kx = 0u, kn = 0xFFFFFFFFu;  // range of the live keys
    for (int j = lane; j < st.cnt; j += 64) {
        const float v = bv[j];
        alive += (v >= tau_est);
        if (v == v) {
            kx = max(kx, fkey(v));
            kn = min(kn, fkey(v));
        }
    }
    alive = wave_sum(alive);
    kx = wave_max_u(kx);
    kn = wave_min_u(kn);
    if (lane == 0) {
        S.wcnt[w] = st.cnt;
        S.walive[w] = alive;
        S.wtau[w] = st.tau;
        S.wstrict[w] = st.strict;
        S.wkmax[w] = kx;
        S.wkmin[w] = kn;
    }
    __syncthreads();
    {
        int tot = 0, strict_any = 0;
#pragma unroll
        for (int ww = 0; ww < NWAVE; ++ww) {
            tot += S.walive[ww];
            strict_any |= S.wstrict[ww];
        }
        if (tau_est == -INFINITY || strict_any || tot >= k || S.nan_flag) break;
        tau_est = -INFINITY;
    }
    }  // attempt
    if (LIST) {
        // the head's per-row state starts from zero at its next launch
        if (tid < 64) A.hslots[(size_t)b * 64 + tid] = 0u;
        if (tid <= HSUB) A.hmeta[(size_t)b * HMETA_STRIDE + tid] = int4{0, 0, 0, 0};
    }

    // Past the stream.  The arguments are read again from the kernel argument
    // segment through an opaque pointer, so that the fields the rest of the
    // row needs (outputs, epilogue parameters, slice lists) are loaded here
    // instead of being held in scalar registers across the stream loop.
    {
    typedef __attribute__((address_space(4))) const KArgs *KArgsConst;
    KArgsConst kargs = (KArgsConst)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(kargs));
    const KArgs &A = *(const KArgs *)kargs;

    if (nsl > 1) {
        // ---- slice: publish the values that can reach the row's pool -------
        // The slice's own k-th largest Ts is a lower bound of the row's, so
        // every slice value >= the row threshold is >= Ts.  The list holds
        // the values passing (ltau, lstrict): >= Ts normally; > t* when a wave
        // kept only values above its threshold t* >= Ts (ties beyond its
        // buffer) or when the ties at Ts exceed the list capacity; every value
        // of the slice when it has fewer than k.
        int tot_s = 0, strict_s = 0;
        float tstar_s = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < NWAVE; ++ww) {
            tot_s += S.walive[ww];
            if (S.wstrict[ww]) {
                strict_s = 1;
                tstar_s = fmaxf(tstar_s, S.wtau[ww]);
            }
        }
        float ltau = -INFINITY;
        bool lstrict = false;
        const int cnt_w = S.wcnt[w];
        int mine = 0, n_s = 0, off = 0;
        bool listed = false;
        if (k <= 64 && !strict_s && tot_s >= k) {
            // A cheaper cut first: the k-th largest L of the 256 lanes' largest
            // entries is at most the slice's k-th largest (k distinct entries
            // reach it), so the entries >= L hold every value that can reach
            // the row's pool; used when they fit the list.
            unsigned *lkeys = S.u.h.whist[0];
            uint32_t lm = 0u;
            for (int j = lane; j < cnt_w; j += 64) {
                const float v = bv[j];
                if (v == v) lm = max(lm, fkey(v));
            }
            lkeys[tid] = lm;
            __syncthreads();
            if (w == 0) {
                const uint32_t q0 = lkeys[lane], q1 = lkeys[64 + lane], q2 = lkeys[128 + lane],
                               q3 = lkeys[192 + lane];
                uint32_t K = 0u;
                for (int bit = 31; bit >= 0; --bit) {
                    const uint32_t cand = K | (1u << bit);
                    const int c = __popcll(__ballot(q0 >= cand)) + __popcll(__ballot(q1 >= cand)) +
                                  __popcll(__ballot(q2 >= cand)) + __popcll(__ballot(q3 >= cand));
                    if (c >= k) K = cand;
                }
                if (lane == 0) S.sel_rem = (int)K;
            }
            __syncthreads();
            const uint32_t L = (uint32_t)S.sel_rem;
            if (L) {
                const float lf = keyf(L);
#pragma unroll
                for (int r = 0; r < PER; ++r) {
                    const int j = lane + 64 * r;
                    mine += (j < cnt_w) && passes(bv[j], lf, false);
                }
                off = block_excl_scan(mine, n_s, S.wsum[0]);
                if (n_s <= A.lcap) {
                    ltau = lf;
                    listed = true;
                }
            }
        }
        if (!listed) {
            float Ts = -INFINITY;
            if (tot_s >= k) {
                uint32_t kn, kx;
                block_key_range(S, kn, kx);
                Ts = keyf(block_kth_union<CAPW>(S, k, kn, kx));
            }
            if (strict_s && (tot_s < k || Ts <= tstar_s)) {
                ltau = tstar_s;
                lstrict = true;
            } else if (tot_s >= k) {
                ltau = Ts;
            }
            mine = 0;
#pragma unroll
            for (int r = 0; r < PER; ++r) {
                const int j = lane + 64 * r;
                mine += (j < cnt_w) && passes(bv[j], ltau, lstrict);
            }
            off = block_excl_scan(mine, n_s, S.wsum[1]);
        }
        if (n_s > A.lcap) {
            // more ties at Ts than the list holds (fewer than k values lie above)
            lstrict = true;
            mine = 0;
#pragma unroll
            for (int r = 0; r < PER; ++r) {
                const int j = lane + 64 * r;
                mine += (j < cnt_w) && passes(bv[j], ltau, true);
            }
            off = block_excl_scan(mine, n_s, S.wsum[0]);
        }
        // (fewer than k values lie above Ts or t*, and lcap > k; a list that
        // would still not fit is reported instead of written)
        const bool overflow = n_s > A.lcap;
        const size_t lo = ((size_t)b * nsl + sl) * A.lcap;
        // The list and its metadata are written and read with device-coherent
        // (agent-scope) accesses, and every thread's writes have completed
        // (vmcnt 0) before the arrival is counted.  Release/acquire fences
        // would instead write back and invalidate the whole L2 of the XCD for
        // every slice.
        if (!overflow) {
#pragma unroll
            for (int r = 0; r < PER; ++r) {
                const int j = lane + 64 * r;
                if (j < cnt_w && passes(bv[j], ltau, lstrict)) {
                    dev_store(A.lst_val + lo + off, bv[j]);
                    dev_store(A.lst_idx + lo + off, bi[j]);
                    off++;
                }
            }
        }
        if (tid == 0) {
            int *m = reinterpret_cast<int *>(A.lst_meta + (size_t)b * nsl + sl);
            dev_store(m + 0, overflow ? 0 : n_s);
            dev_store(m + 1, (int)__float_as_uint(ltau));
            dev_store(m + 2, lstrict ? 1 : 0);
            dev_store(m + 3, (overflow ? 1 : 0) | (S.nan_flag ? 2 : 0));
        }
        wait_stores_done();
        __syncthreads();
        if (tid == 0) S.sel_rem = (int)atomicAdd(&A.arrive[b], 1u);
        __syncthreads();
        if (S.sel_rem != nsl - 1) return;

        // ---- finisher: gather every slice's list ---------------------------
        // into the wave-buffer layout (entry i of the concatenation at
        // cval[i]: wave w holds [w*CAPW, w*CAPW + wcnt[w]))
        int *offs = reinterpret_cast<int *>(S.u.h.whist[0]);  // nsl + 1 ints
        float *mtau = reinterpret_cast<float *>(S.u.h.whist[1]);
        int *mstr = reinterpret_cast<int *>(S.u.h.whist[2]);
        if (w == 0) {
            int cnt = 0, st = 0, ov = 0;
            float tv = -INFINITY;
            if (lane < nsl) {
                const int *m = reinterpret_cast<const int *>(A.lst_meta + (size_t)b * nsl + lane);
                cnt = min(max(dev_load(m + 0), 0), A.lcap);
                tv = __uint_as_float((uint32_t)dev_load(m + 1));
                st = dev_load(m + 2);
                ov = dev_load(m + 3);
            }
            const int incl = wave_incl_scan(cnt);
            if (lane < nsl) {
                offs[lane] = incl - cnt;
                mtau[lane] = tv;
                mstr[lane] = st;
            }
            if (lane == 63) offs[MAX_SLICES] = incl;
            const bool any_ov = __ballot(ov & 1) != 0ull;
            const bool any_nan = __ballot(ov & 2) != 0ull;
            if (lane == 0) {
                offs[MAX_SLICES + 1] = any_ov ? 1 : 0;
                S.nan_flag = any_nan ? 1 : 0;
            }
        }
        __syncthreads();
        const int ntot = offs[MAX_SLICES];
        if (offs[MAX_SLICES + 1]) {
            // A slice list did not fit.  Unreachable: a list holds either
            // values >= a slice's k-th largest when they fit, or values strictly
            // above it (or above a wave's tie threshold t* >= it), of which
            // there are fewer than k, and the host keeps lcap > k.  Reported as
            // token -1 (documented as an internal error) rather than sampled.
            if (tid == 0) {
                A.out_token[b] = -1;
                if (A.out_ncand) A.out_ncand[b] = -1;
                A.arrive[b] = 0u;
            }
            return;
        }
        uint32_t kx = 0u, kn = 0xFFFFFFFFu;
        // every list at once (entry i of the concatenation -> its list j by
        // the offsets), so that all loads are in flight together
        for (int i = tid; i < ntot; i += WG) {
            int j = 0;
            while (j + 1 < nsl && offs[j + 1] <= i) ++j;
            const size_t src = ((size_t)b * nsl + j) * A.lcap + (i - offs[j]);
            const float v = dev_load(A.lst_val + src);
            S.cval[i] = v;
            S.cidx[i] = dev_load(A.lst_idx + src);
            if (v == v) {
                kx = max(kx, fkey(v));
                kn = min(kn, fkey(v));
            }
        }
        kx = wave_max_u(kx);
        kn = wave_min_u(kn);
        if (lane == 0) {
            S.wkmax[w] = kx;  // partial ranges: only their union is used
            S.wkmin[w] = kn;
        }
        if (tid < NWAVE) {
            const int c = min(max(ntot - tid * CAPW, 0), CAPW);
            S.wcnt[tid] = c;
            S.walive[tid] = c;
            int any = 0;
            float ts = -INFINITY;
            if (tid == 0) {
                for (int j = 0; j < nsl; ++j)
                    if (mstr[j]) {
                        any = 1;
                        ts = fmaxf(ts, mtau[j]);
                    }
            }
            S.wstrict[tid] = any;
            S.wtau[tid] = ts;
        }
        if (tid == 0) A.arrive[b] = 0u;
        __syncthreads();
    }

    // ---- exact threshold over the union of the wave buffers ---------------
    int total = 0, any_strict = 0;
    float tstar = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < NWAVE; ++ww) {
        total += S.walive[ww];
        if (S.wstrict[ww]) {
            any_strict = 1;
            tstar = fmaxf(tstar, S.wtau[ww]);
        }
    }
    float T = -INFINITY;
    bool rescan = false;
    int nc = 0, off = 0;
    int forced_token = -1;
    const bool nan_row = S.nan_flag != 0;
    bool nan_first = false;
    if (nan_row && A.greedy) {
        const float y0 = rescan_value<HAS_BIAS, HAS_ALLOW>(A, S, row, abits, use_hash, 0);
        nan_first = y0 != y0;
    }
    if (nan_row && !A.greedy) {
        // A nan compares false with everything, so the reference heap's
        // threshold depends on where the nan entered it: replay the heap
        T = heap_replay_threshold<HAS_BIAS, HAS_ALLOW>(A, S, R, k);
        rescan = true;
    } else if (nan_first) {
        // the greedy scan (best = 0; later ids win only when strictly larger)
        // keeps id 0 when its value is nan; otherwise nan never wins and the
        // k = 1 selection below is exact
        T = NAN;
        forced_token = 0;
        rescan = true;
    } else if (HAS_BIAS && nan_row) {
        // a nan bias maximum makes every flagged entry's stream bound a nan,
        // so the buffers can lack the row's maximum: the scan's best is the
        // root of a one-entry heap fed in id order (id 0 is not a nan here,
        // and a nan never replaces the root), found over the exact values
        T = heap_replay_threshold<HAS_BIAS, HAS_ALLOW>(A, S, R, 1);
        rescan = true;
    } else if (total >= k) {
        uint32_t kn, kx;
        block_key_range(S, kn, kx);
        T = keyf(block_kth_union<CAPW>(S, k, kn, kx));
        if (any_strict && T <= tstar) {
            T = tstar;
            rescan = true;
        }
    } else if (any_strict) {
        T = tstar;
        rescan = true;
    }

    const bool top_p_on = (A.top_p > 0.0f && A.top_p < 1.0f) && !A.greedy;
    // the row's uniform, read only now that the stream's registers are free
    const float uu = (A.uniforms && !A.greedy) ? A.uniforms[b] : 0.0f;
    int token = V - 1;
    int n_cand = 0, n_kept = 0;
    float sum2 = 0.0f;

    // ---- the pool (>= T) of every wave buffer --------------------------
    float rv[PER];
    int ri[PER];
    if (!rescan) {
        int mine = 0;
        const int cnt_w = S.wcnt[w];
#pragma unroll
        for (int r = 0; r < PER; ++r) {
            const int j = lane + 64 * r;  // own wave's buffer
            rv[r] = (j < cnt_w) ? bv[j] : NAN;
            ri[r] = (j < cnt_w) ? bi[j] : -1;
            mine += (rv[r] >= T);
        }
        off = block_excl_scan(mine, nc, S.wsum[0]);
        if (nc > EP_ALL) rescan = true;  // epilogue scratch too small: id-order rescan
    }

    if (!rescan) {
        // ---- compact the pool to the front, then sort by id ---------------
        __syncthreads();
        int pos = off;
#pragma unroll
        for (int r = 0; r < PER; ++r) {
            if (rv[r] >= T) {
                S.cval[pos] = rv[r];
                S.cidx[pos] = ri[r];
                pos++;
            }
        }
        __syncthreads();
        n_cand = nc;
        if (nc <= 64) {
            // one candidate per lane of wave 0; ranks against all 64 slots read
            // four at a time, slots past the pool holding INT_MAX (no barrier)
            if (w == 0) {
                const float myv = (lane < nc) ? S.cval[lane] : 0.0f;
                const int myid = (lane < nc) ? S.cidx[lane] : INT_MAX;
                if (lane >= nc) S.cidx[lane] = INT_MAX;
                wave_sync();
                int rank = 0;
                for (int q4 = 0; q4 < ((nc + 3) >> 2); ++q4) {
                    const int4 v = reinterpret_cast<const int4 *>(S.cidx)[q4];
                    rank += (v.x < myid) + (v.y < myid) + (v.z < myid) + (v.w < myid);
                }
                wave_sync();
                if (lane < nc) {
                    S.cval[rank] = myv;
                    S.cidx[rank] = myid;
                }
                wave_sync();
            }
        } else if (2 * nc <= NWAVE * CAPW) {
            // bucket sort by id (ids in the pool are distinct): buckets of
            // 2^sh ids (at most EP_ALL / 2 of them) are counted and scanned
            // in the epilogue scratch, the entries dealt into their buckets
            // at [nc, 2 nc) of the buffers, and each entry's place is its
            // bucket's start plus the ids below it in the bucket (a few)
            int rk_b[PER];
            int sh = 8;
            while (((V - 1) >> sh) >= EP_ALL / 2) ++sh;
            const int nbk = ((V - 1) >> sh) + 1;
            int *bcnt = reinterpret_cast<int *>(S.u.ep);
            int *boff = bcnt + EP_ALL / 2;
            for (int i = tid; i < nbk; i += WG) bcnt[i] = 0;
            __syncthreads();
#pragma unroll
            for (int r = 0; r < PER; ++r) {
                const int j = tid + r * WG;
                if (j < nc) {
                    rv[r] = S.cval[j];
                    ri[r] = S.cidx[j];
                    atomicAdd(&bcnt[ri[r] >> sh], 1);
                }
            }
            __syncthreads();
            // exclusive scan of the counts: thread t owns buckets
            // [t * BPT, t * BPT + BPT)
            constexpr int BPT = (EP_ALL / 2 + WG - 1) / WG;
            int lsum = 0;
#pragma unroll
            for (int q = 0; q < BPT; ++q) {
                const int bk = tid * BPT + q;
                lsum += (bk < nbk) ? bcnt[bk] : 0;
            }
            int btot = 0;
            int run = block_excl_scan(lsum, btot, S.wsum[0]);
#pragma unroll
            for (int q = 0; q < BPT; ++q) {
                const int bk = tid * BPT + q;
                if (bk < nbk) {
                    boff[bk] = run;
                    run += bcnt[bk];
                }
            }
            __syncthreads();
            float *tv = S.cval + nc;
            int *ti = S.cidx + nc;
#pragma unroll
            for (int r = 0; r < PER; ++r) {
                if (tid + r * WG < nc) {
                    const int pos = atomicAdd(&boff[ri[r] >> sh], 1);
                    tv[pos] = rv[r];
                    ti[pos] = ri[r];
                }
            }
            __syncthreads();
            // boff now holds each bucket's end
#pragma unroll
            for (int r = 0; r < PER; ++r) {
                const int pidx = tid + r * WG;
                if (pidx < nc) {
                    const int id = ti[pidx];
                    const int bk = id >> sh;
                    const int end = boff[bk], start = end - bcnt[bk];
                    int rank = start;
                    for (int q = start; q < end; ++q) rank += (ti[q] < id);
                    rv[r] = tv[pidx];
                    ri[r] = id;
                    rk_b[r] = rank;
                }
            }
            __syncthreads();
#pragma unroll
            for (int r = 0; r < PER; ++r) {
                if (tid + r * WG < nc) {
                    S.cval[rk_b[r]] = rv[r];
                    S.cidx[rk_b[r]] = ri[r];
                }
            }
            __syncthreads();
        } else {
            int rk[PER];
#pragma unroll
            for (int r = 0; r < PER; ++r) {
                const int j = tid + r * WG;
                rk[r] = -1;
                if (j < nc) {
                    rv[r] = S.cval[j];
                    ri[r] = S.cidx[j];
                    // eight slots per round, so that eight LDS reads are in
                    // flight rather than one
                    int rank = 0, q = 0;
                    for (; q + 8 <= nc; q += 8) {
#pragma unroll
                        for (int u = 0; u < 8; ++u) rank += (S.cidx[q + u] < ri[r]);
                    }
                    for (; q < nc; ++q) rank += (S.cidx[q] < ri[r]);
                    rk[r] = rank;
                }
            }
            __syncthreads();
#pragma unroll
            for (int r = 0; r < PER; ++r) {
                if (rk[r] >= 0) {
                    S.cval[rk[r]] = rv[r];
                    S.cidx[rk[r]] = ri[r];
                }
            }
            __syncthreads();
        }

        if (nc == 0) {
            // no value reaches the threshold: the softmax sum is 0, so the
            // filtered variant's argmax over nothing gives 0, the draw r = 0
            token = (A.variant == LAL_GPU_VARIANT_FILTERED || (A.flags & LAL_GPU_F_DRAW_GPT2)) ? 0 : A.fallback;
        } else if (A.greedy) {
            if (nc <= 64) __syncthreads();  // wave 0 sorted the pool
            token = S.cidx[0];
            if ((A.flags & LAL_GPU_F_GREEDY_FILTER) && is_banned(S, 0)) token = 0;
            n_kept = 1;
            for (int j = tid; j < nc && j < A.cand_ld; j += WG) {
                const size_t o = (size_t)b * A.cand_ld + j;
                const bool kept = S.cidx[j] == token;
                if (A.cand_ids) A.cand_ids[o] = S.cidx[j];
                if (A.cand_vals) A.cand_vals[o] = S.cval[j];
                if (A.cand_kept) A.cand_kept[o] = kept ? 1 : 0;
                if (A.cand_probs) A.cand_probs[o] = kept ? 1.0f : 0.0f;
            }
        } else if (nc <= 64) {
            if (w == 0) {
                const RowResult rr = wave_epilogue(A, S, nc, uu, b);
                token = rr.token;
                n_kept = rr.n_kept;
                sum2 = rr.sum;
            }
        } else {
            const RowResult rr = block_epilogue<PER>(A, S, nc, uu, b);
            token = rr.token;
            n_kept = rr.n_kept;
            sum2 = rr.sum;
        }
    } else {
        // ---- rescan: the pool is larger than the LDS buffers --------------
        Nucleus N;
        N.on = false;
        N.amax = N.inv = N.plim = 0.0f;
        N.idlim = 0;
        bool use_ban = A.any_bans && !A.greedy;
        if (top_p_on) {
            const RescanStats pool = rescan_stats<HAS_BIAS, HAS_ALLOW>(A, S, row, abits, use_hash, T,
                                                                       false, N);
            N = rescan_nucleus<HAS_BIAS, HAS_ALLOW>(A, S, row, abits, use_hash, T, pool.n_cand,
                                                    pool.max_kept);
        }
        RescanStats rs = rescan_stats<HAS_BIAS, HAS_ALLOW>(A, S, row, abits, use_hash, T, use_ban, N);
        if (rs.n_kept == 0 && (use_ban || N.on)) {
            // restore the whole top-k pool
            use_ban = false;
            N.on = false;
            rs = rescan_stats<HAS_BIAS, HAS_ALLOW>(A, S, row, abits, use_hash, T, false, N);
        }
        n_cand = rs.n_cand;
        n_kept = rs.n_kept;
        if (A.greedy) {
            token = (forced_token >= 0) ? forced_token : rs.first_kept;
            if ((A.flags & LAL_GPU_F_GREEDY_FILTER) && is_banned(S, 0)) token = 0;
            n_kept = 1;
            if (A.cand_ld > 0)
                rescan_write_cands<HAS_BIAS, HAS_ALLOW>(A, S, row, abits, use_hash, T, false, N, 0.0f,
                                                        1.0f, true, token, b);
        } else {
            const float mx = (rs.max_kept > -1e30f) ? rs.max_kept : -1e30f;
            sum2 = rescan_sequential<HAS_BIAS, HAS_ALLOW>(A, S, row, abits, use_hash, T, use_ban, N, mx,
                                                          false, 0.0f, nullptr);
            if (A.variant == LAL_GPU_VARIANT_FILTERED && sum2 <= 0.0f) {
                token = (rs.max_kept > -1e30f) ? rs.first_max_kept : 0;
            } else {
                const float rr = uu * sum2;
                if ((A.flags & LAL_GPU_F_DRAW_GPT2) && rr == 0.0f) {
                    token = 0;
                } else {
                    int f = -1;
                    rescan_sequential<HAS_BIAS, HAS_ALLOW>(A, S, row, abits, use_hash, T, use_ban, N,
                                                           mx, true, rr, &f);
                    token = (f < 0) ? A.fallback : f;
                }
            }
            if (A.cand_ld > 0)
                rescan_write_cands<HAS_BIAS, HAS_ALLOW>(A, S, row, abits, use_hash, T, use_ban, N, mx,
                                                        sum2, false, token, b);
        }
    }

    if (tid == 0) {
        A.out_token[b] = token;
        if (A.out_thr) A.out_thr[b] = T;
        if (A.out_ncand) A.out_ncand[b] = n_cand;
        if (A.out_nkept) A.out_nkept[b] = n_kept;
        if (A.out_sum) A.out_sum[b] = sum2;
    }

    // ---- in-place penalty side effect / penalised history values --------
    if ((A.flags & LAL_GPU_F_WRITEBACK) || A.out_hvals) {
        __syncthreads();
        float *pv = S.u.h.hval;
        for (int s = tid; s < HSLOTS; s += WG) {
            const int key = S.hkey[s];
            if (key >= 0) pv[s] = penalise(row[key], S.hinfo[s] & HCOUNT_MASK, A.pen);
        }
        __syncthreads();
        if (A.out_hvals) {
            for (int i = tid; i < nh; i += WG) {
                const int t = hrow[i];
                if (t >= 0 && t < V) A.out_hvals[(size_t)b * A.hist_ld + i] = pv[hash_find(S.hkey, t)];
            }
        }
        if (A.flags & LAL_GPU_F_WRITEBACK) {
            for (int s = tid; s < HSLOTS; s += WG) {
                const int key = S.hkey[s];
                if (key >= 0 && (S.hinfo[s] & HCOUNT_MASK)) A.logits_w[(size_t)b * A.ld + key] = pv[s];
            }
        }
    }
    }  // arguments read again
}

// ---------------------------------------------------------------------------
// Finish over a host-filtered pool (tools/server/qwen7b_server.c:268-294,
// after the lal_filter_topk plugin has cleared entries of the keep mask): the
// pool ids ascending with their processed logits, a keep flag per entry; the
// pool is restored when no entry is kept; softmax over the kept entries in id
// order, argmax without a draw when the sum is <= 0 (filtered variant), else
// the first kept id whose running sum reaches u*sum.
// ---------------------------------------------------------------------------
struct FinishArgs {
    int V, variant;
    unsigned flags;
    float T;
    int cand_ld;
    const int *n_cand;
    const int *ids;
    const float *vals;
    const uint8_t *keep;
    const float *uniforms;
    int *out_token, *out_n_kept;
    float *out_sum;
};

struct FSmem {
    float ep[RS_CHUNK];
    float redf[NWAVE];
    int redi[NWAVE];
    int redi2[NWAVE];
    int wsum[2][NWAVE];
    uint64_t exptab[32];
};

__global__ __launch_bounds__(WG) void finish_rows_kernel(FinishArgs F)
{
    __shared__ FSmem S;
    const int b = blockIdx.x, tid = threadIdx.x;
    if (tid < 32) S.exptab[tid] = kExp2Tab[tid];
    const int n = F.n_cand[b];
    const size_t o = (size_t)b * F.cand_ld;
    if (n < 0 || n > F.cand_ld) {  // pool not captured in full
        if (tid == 0) {
            F.out_token[b] = -1;
            if (F.out_n_kept) F.out_n_kept[b] = -1;
        }
        return;
    }
    // keep: 0 dropped, 1 kept pool entry, 2 kept entry outside the pool (it
    // counts for "anything kept" and for the sum <= 0 argmax, not the softmax)
    int nk = 0, na = 0;
    float mk = -INFINITY, ma = -INFINITY;
    for (int i = tid; i < n; i += WG) {
        const uint8_t k = F.keep[o + i];
        const float x = F.vals[o + i];
        nk += (k == 1) ? 1 : 0;
        na += k ? 1 : 0;
        if (k == 1) mk = fmaxf(mk, x);
        if (k) ma = fmaxf(ma, x);
    }
    nk = block_sum(S, nk);
    na = block_sum(S, na);
    const bool restore = (na == 0);  // nothing kept: the whole pool
    if (restore) {
        mk = -INFINITY;
        for (int i = tid; i < n; i += WG) mk = fmaxf(mk, F.vals[o + i]);
    }
    const float kmax = block_max(S, mk);
    const float amax = restore ? kmax : block_max(S, ma);
    const float mx = (kmax > -1e30f) ? kmax : -1e30f;
    // sequential sum in id order, RS_CHUNK entries at a time
    float acc = 0.0f;
    for (int c0 = 0; c0 < n; c0 += RS_CHUNK) {
        const int m = min(RS_CHUNK, n - c0);
        __syncthreads();
        for (int i = tid; i < m; i += WG) {
            const bool kp = restore || F.keep[o + c0 + i] == 1;
            S.ep[i] = kp ? glibc_expf((F.vals[o + c0 + i] - mx) / F.T, S.exptab) : -1.0f;
        }
        acc = block_seq_prefix(S, S.ep, m, acc);
    }
    const float sum = acc;
    int token = (F.flags & LAL_GPU_F_FALLBACK_ZERO) ? 0 : F.V - 1;
    if (F.variant == LAL_GPU_VARIANT_FILTERED && sum <= 0.0f) {
        // first id of the largest kept value above -1e30 (ids of entries
        // outside the pool need not be in order)
        int first = INT_MAX;
        for (int i = tid; i < n; i += WG)
            if ((restore || F.keep[o + i]) && F.vals[o + i] == amax && amax > -1e30f)
                first = min(first, F.ids[o + i]);
        first = block_min(S, first);
        token = (first == INT_MAX) ? 0 : first;
    } else {
        const float r = (F.uniforms ? F.uniforms[b] : 0.0f) * sum;
        if ((F.flags & LAL_GPU_F_DRAW_GPT2) && r == 0.0f) {
            token = 0;
        } else {
            float run = 0.0f;
            for (int c0 = 0; c0 < n; c0 += RS_CHUNK) {
                const int m = min(RS_CHUNK, n - c0);
                __syncthreads();
                for (int i = tid; i < m; i += WG) {
                    const bool kp = restore || F.keep[o + c0 + i] == 1;
                    S.ep[i] = kp ? glibc_expf((F.vals[o + c0 + i] - mx) / F.T, S.exptab) : -1.0f;
                }
                run = block_seq_prefix(S, S.ep, m, run);
                int first = INT_MAX;
                for (int i = tid; i < m; i += WG) {
                    const bool kp = restore || F.keep[o + c0 + i] == 1;
                    if (kp && r <= S.ep[i]) first = min(first, i);
                }
                first = block_min(S, first);
                if (first != INT_MAX) {
                    token = F.ids[o + c0 + first];
                    break;
                }
            }
        }
    }
    if (tid == 0) {
        F.out_token[b] = token;
        if (F.out_n_kept) F.out_n_kept[b] = restore ? n : nk;
        if (F.out_sum) F.out_sum[b] = sum;
    }
}

// ---------------------------------------------------------------------------
// int8 LM head front end (runtime/lal_q8_kernel.h:375-543)
// ---------------------------------------------------------------------------
// x86 float -> int32 conversion as the reference's builds execute it
// (cvtps2dq rounds to nearest even, a C cast truncates): a nan or a value
// outside the int32 range gives INT_MIN
__device__ __forceinline__ int x86_cvt(float v, bool round_even)
{
    if (!(v >= -2147483648.0f && v < 2147483648.0f)) return INT_MIN;
    return round_even ? (int)__builtin_rintf(v) : (int)v;
}

// _mm_max_ps: the first operand if it is greater, else the second
__device__ __forceinline__ float x86_maxps(float a, float b) { return (a > b) ? a : b; }

// Scale of one activation row as lal_quantize_x_int8 computes it, for one
// 256-thread block (every thread calls it; barriers inside).  mode 0 (AVX2
// build): lane j of the 8-wide maximum sees |x[8c + j]| in chunk order, and a
// nan there is kept only while no later value of the lane follows, so thread
// (segment s, lane j) folds its run of chunks into (nan seen, ends in nan,
// maximum after its last nan) and lane j's 32 runs are folded in order; the
// lanes then reduce as the build's shuffles do, and the tail is folded in with
// `a > max`.  mode 1: `a > max` over all values, which never takes a nan.
struct QxShared {
    float seg_m[256];
    int seg_f[256];
    float red[4];
};

__device__ float qx_scale(const float *xr, int n, int mode, QxShared &Q)
{
    const int t = threadIdx.x;
    float m = 0.0f;
    if (mode == 0) {
        const int n8 = n & ~7;
        const int j = t & 7, sgi = t >> 3, nch = n8 >> 3;
        const int c0 = (int)(((long long)nch * sgi) / 32), c1 = (int)(((long long)nch * (sgi + 1)) / 32);
        float acc = -1.0f;  // -1: no value after the last nan
        int f = 0;          // 1: a nan seen, 2: the run ends in a nan, 4: the run has values
        for (int c = c0; c < c1; ++c) {
            const float a = fabsf(xr[8 * c + j]);
            if (a != a) {
                f = 1 | 2 | 4;
                acc = -1.0f;
            } else {
                f = (f & 1) | 4;
                acc = fmaxf(acc, a);
            }
        }
        __syncthreads();  // Q is free (an earlier call's readers are done)
        Q.seg_m[t] = acc;
        Q.seg_f[t] = f;
        __syncthreads();
        if (t < 8) {
            float la = -1.0f;
            int lf = 0;
            for (int sg = 0; sg < 32; ++sg) {
                const int ff = Q.seg_f[sg * 8 + t];
                if (!(ff & 4)) continue;
                if (ff & 1) {
                    lf = ff;
                    la = Q.seg_m[sg * 8 + t];
                } else {
                    lf = (lf & 1) | 4;
                    la = fmaxf(la, Q.seg_m[sg * 8 + t]);
                }
            }
            Q.seg_m[t] = (lf & 2) ? __builtin_nanf("") : fmaxf(la, 0.0f);
        }
        __syncthreads();
        if (t == 0) {
            float h[4];
            for (int q = 0; q < 4; ++q) h[q] = x86_maxps(Q.seg_m[q], Q.seg_m[q + 4]);
            const float s1[4] = {h[2], h[3], h[0], h[1]};
            for (int q = 0; q < 4; ++q) h[q] = x86_maxps(h[q], s1[q]);
            float mm = x86_maxps(h[0], h[1]);
            for (int i = n8; i < n; ++i) {
                const float a = fabsf(xr[i]);
                if (a > mm) mm = a;
            }
            Q.red[0] = mm;
        }
        __syncthreads();
        m = Q.red[0];
    } else {
        for (int i = t; i < n; i += 256) m = fmaxf(m, fabsf(xr[i]));
        m = wave_max(m);
        __syncthreads();
        if (lane_id() == 0) Q.red[wave_id()] = m;
        __syncthreads();
        m = fmaxf(fmaxf(Q.red[0], Q.red[1]), fmaxf(Q.red[2], Q.red[3]));
    }
    float scale = m / 127.0f;
    if (scale < 1e-8f) scale = 1e-8f;
    return scale;
}

// q of x[i] (i < n8: rounded, else truncated), x86 conversion, clamped
__device__ __forceinline__ int8_t qx_value(float x, float inv, bool round_even)
{
    return (int8_t)min(127, max(-127, x86_cvt(x * inv, round_even)));
}

__global__ __launch_bounds__(256) void quantize_x_kernel(const float *x, int n, int mode,
                                                         int8_t *xq, float *sx)
{
    __shared__ QxShared Q;
    const int b = blockIdx.x, t = threadIdx.x;
    const float *xr = x + (size_t)b * n;
    const float scale = qx_scale(xr, n, mode, Q);
    const float inv = 1.0f / scale;
    const int n8 = (mode == 0) ? (n & ~7) : 0;
    for (int i = t; i < n; i += 256) xq[(size_t)b * n + i] = qx_value(xr[i], inv, i < n8);
    if (t == 0) sx[b] = scale;
}

// quantize_x_kernel for rows of at most 4096 values, in one round trip: each
// thread loads its values once (thread (segment s, lane j) holds x[8c + j]
// for the chunks c of segment s, as qx_scale folds them), the per-lane folds
// of the AVX2 build combine across segments with shuffles (the fold is
// associative: a run that holds a nan replaces what precedes it, one without
// keeps the earlier nan flag and takes the larger maximum), and the bytes
// leave through LDS in 16-byte stores.  Same values as quantize_x_kernel.
constexpr int QXF_MAXN = 4096;
constexpr int QXF_PT = QXF_MAXN / 256;  // chunks per segment at most

__global__ __launch_bounds__(256) void quantize_x_fast_kernel(const float *x, int n, int mode, int8_t *xq,
                                                              float *sx)
{
    __shared__ float seg_m[4][8];
    __shared__ int seg_f[4][8];
    __shared__ float lane_m[8];
    __shared__ float tailv[8];
    __shared__ float red[4];
    __shared__ __align__(16) int8_t qs[QXF_MAXN];
    const int b = blockIdx.x, t = threadIdx.x, lane = lane_id(), wv = wave_id();
    const float *xr = x + (size_t)b * n;
    const int n8 = n & ~7, nch = n8 >> 3;
    const int j = t & 7, sgi = t >> 3;
    const int c0 = (int)(((long long)nch * sgi) / 32), c1 = (int)(((long long)nch * (sgi + 1)) / 32);
    float v[QXF_PT];
#pragma unroll
    for (int u = 0; u < QXF_PT; ++u) v[u] = xr[min(8 * (c0 + u) + j, n - 1)];  // every load issued
    const int ntail = n - n8;
    const float tv = xr[min(n8 + min(t, 7), n - 1)];
    if (t < ntail) tailv[t] = tv;
    float m = 0.0f;
    if (mode == 0) {
        float acc = -1.0f;  // -1: no value after the last nan
        int f = 0;          // 1: a nan seen, 2: the run ends in a nan, 4: the run has values
#pragma unroll
        for (int u = 0; u < QXF_PT; ++u) {
            if (c0 + u < c1) {
                const float a = fabsf(v[u]);
                if (a != a) {
                    f = 1 | 2 | 4;
                    acc = -1.0f;
                } else {
                    f = (f & 1) | 4;
                    acc = fmaxf(acc, a);
                }
            }
        }
        // segments 8w .. 8w+7 of lane j sit in lanes j, j+8, .., j+56 of wave
        // w: fold them in order, the later run on the right
#pragma unroll
        for (int off = 8; off < 64; off <<= 1) {
            const int rf = __shfl_down(f, off, 64);
            const float racc = __shfl_down(acc, off, 64);
            if ((lane & (2 * off - 1)) < 8 && (rf & 4)) {
                if (rf & 1) {
                    f = rf;
                    acc = racc;
                } else {
                    f = (f & 1) | 4;
                    acc = fmaxf(acc, racc);
                }
            }
        }
        if (lane < 8) {
            seg_m[wv][lane] = acc;
            seg_f[wv][lane] = f;
        }
        __syncthreads();
        if (t < 8) {
            float la = -1.0f;
            int lf = 0;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const int ff = seg_f[w][t];
                if (!(ff & 4)) continue;
                if (ff & 1) {
                    lf = ff;
                    la = seg_m[w][t];
                } else {
                    lf = (lf & 1) | 4;
                    la = fmaxf(la, seg_m[w][t]);
                }
            }
            lane_m[t] = (lf & 2) ? __builtin_nanf("") : fmaxf(la, 0.0f);
        }
        __syncthreads();
        if (t == 0) {
            // the build's lane reduction (_mm256 halves, then shuffles), then
            // the tail with `a > max`
            float h[4];
            for (int q = 0; q < 4; ++q) h[q] = x86_maxps(lane_m[q], lane_m[q + 4]);
            const float s1[4] = {h[2], h[3], h[0], h[1]};
            for (int q = 0; q < 4; ++q) h[q] = x86_maxps(h[q], s1[q]);
            float mm = x86_maxps(h[0], h[1]);
            for (int i = 0; i < ntail; ++i) {
                const float a = fabsf(tailv[i]);
                if (a > mm) mm = a;
            }
            red[0] = mm;
        }
        __syncthreads();
        m = red[0];
    } else {
        // `a > max` over every value: order-free, never a nan
#pragma unroll
        for (int u = 0; u < QXF_PT; ++u)
            if (c0 + u < c1) m = fmaxf(m, fabsf(v[u]));
        if (t < ntail) m = fmaxf(m, fabsf(tv));
        m = wave_max(m);
        if (lane == 0) red[wv] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    }
    float scale = m / 127.0f;
    if (scale < 1e-8f) scale = 1e-8f;
    const float inv = 1.0f / scale;
    // mode 0 rounds the 8-wide prefix and truncates the tail; mode 1 truncates
#pragma unroll
    for (int u = 0; u < QXF_PT; ++u)
        if (c0 + u < c1) qs[8 * (c0 + u) + j] = qx_value(v[u], inv, mode == 0);
    if (t < ntail) qs[n8 + t] = qx_value(tv, inv, false);
    __syncthreads();
    int8_t *dst = xq + (size_t)b * n;
    if ((n & 15) == 0 && (((uintptr_t)dst) & 15) == 0) {
        for (int i = t; i < n / 16; i += 256)
            reinterpret_cast<int4 *>(dst)[i] = reinterpret_cast<const int4 *>(qs)[i];
    } else {
        for (int i = t; i < n; i += 256) dst[i] = qs[i];
    }
    if (t == 0) sx[b] = scale;
}

// GEMV/GEMM-by-rows: each wave computes LMH_ROWS vocab rows for all batch rows
// with v_dot4 int8 dot products (exact int32 accumulation).
constexpr int LMH_ROWS = 4;
constexpr int LMH_MAXB = 8;

template <int NB>
__global__ __launch_bounds__(256) void lm_head_dot4_kernel(const int8_t *xq, const float *sx, int n,
                                                           const int8_t *w, const float *sw, int V,
                                                           float *logits, int ld, int b0)
{
    const int wave = blockIdx.x * 4 + wave_id();
    const int v0 = wave * LMH_ROWS;
    if (v0 >= V) return;
    const int lane = lane_id();
    int acc[LMH_ROWS][NB];
#pragma unroll
    for (int r = 0; r < LMH_ROWS; ++r)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[r][j] = 0;
    const int n16 = n >> 4;  // 16-byte chunks
    for (int c = lane; c < n16; c += 64) {
        int4 xv[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j)
            xv[j] = *reinterpret_cast<const int4 *>(xq + (size_t)(b0 + j) * n + 16 * c);
#pragma unroll
        for (int r = 0; r < LMH_ROWS; ++r) {
            if (v0 + r >= V) break;
            const i32x4 wv = __builtin_nontemporal_load(
                reinterpret_cast<const i32x4 *>(w + (size_t)(v0 + r) * n + 16 * c));
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                int a = acc[r][j];
                a = __builtin_amdgcn_sdot4(wv.x, xv[j].x, a, false);
                a = __builtin_amdgcn_sdot4(wv.y, xv[j].y, a, false);
                a = __builtin_amdgcn_sdot4(wv.z, xv[j].z, a, false);
                a = __builtin_amdgcn_sdot4(wv.w, xv[j].w, a, false);
                acc[r][j] = a;
            }
        }
    }
    // tail (n not a multiple of 16)
    for (int i = 16 * n16 + lane; i < n; i += 64) {
#pragma unroll
        for (int r = 0; r < LMH_ROWS; ++r) {
            if (v0 + r >= V) break;
            const int wv = w[(size_t)(v0 + r) * n + i];
#pragma unroll
            for (int j = 0; j < NB; ++j) acc[r][j] += wv * (int)xq[(size_t)(b0 + j) * n + i];
        }
    }
#pragma unroll
    for (int r = 0; r < LMH_ROWS; ++r)
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            int a = acc[r][j];
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) a += __shfl_xor(a, d, 64);
            acc[r][j] = a;
        }
    if (lane < LMH_ROWS * NB) {
        const int r = lane / NB, j = lane % NB;
        int dot = 0;
#pragma unroll
        for (int rr = 0; rr < LMH_ROWS; ++rr)
#pragma unroll
            for (int jj = 0; jj < NB; ++jj)
                if (rr == r && jj == j) dot = acc[rr][jj];
        if (v0 + r < V)
            logits[(size_t)(b0 + j) * ld + v0 + r] = (sx[b0 + j] * sw[v0 + r]) * (float)dot;
    }
}

// Int8 LM head on the matrix cores, for 9..64 batch rows per launch:
// logits[b][v] = (sx[b]*sw[v]) * (float)dot(xq[b], w[v]) with exact int32
// sums (v_mfma_i32_16x16x64_i8; integer products and sums are exact in any
// order).  Operand layout (checked on the device): A = 16 batch rows x 64 k,
// lane l holds row l%16, bytes [16*(l/16), +16); B = 64 k x 16 vocab rows,
// lane l holds row l%16, the same bytes; C = 16 x 16, lane l holds vocab row
// l%16, batch rows 4*(l/16)+i.  Each workgroup owns an equal contiguous range
// of vocab rows and walks it in tiles of 64 (16 per wave), streaming w once
// (three 256-byte passes of k in flight per wave) against the batch's
// activations staged in LDS 256 k-bytes at a time.
constexpr int LMM_WAVES = 4;
constexpr int LMM_TILE_V = 16 * LMM_WAVES;
constexpr int LMM_KC = 256;
constexpr int LMM_MAXB = 64;
typedef int v4i __attribute__((ext_vector_type(4)));

template <int MT>
__global__ __launch_bounds__(64 * LMM_WAVES) void lm_head_mfma_kernel(const int8_t *xq, const float *sx, int n,
                                                                      const int8_t *w, const float *sw, int V,
                                                                      float *logits, int ld, int b0, int nb)
{
    __shared__ __align__(16) int8_t xs[2][MT * 16 * LMM_KC];
    constexpr int XCH = MT * 16 * (LMM_KC / 16);                  // 16-byte chunks per stage
    constexpr int XPT = (XCH + 64 * LMM_WAVES - 1) / (64 * LMM_WAVES);
    const int wv = wave_id(), lane = lane_id(), tid = threadIdx.x;
    const int g = lane >> 4, r16 = lane & 15;
    const int npass = (n + LMM_KC - 1) / LMM_KC;
    const int vlo = (int)(((long long)V * blockIdx.x) / gridDim.x);
    const int vhi = (int)(((long long)V * (blockIdx.x + 1)) / gridDim.x);

    // activations of pass p -> registers (this thread's chunks)
    auto fetch_x = [&](v4i (&xr)[XPT], int p) {
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            const int c = tid + j * 64 * LMM_WAVES;
            const int row = c / (LMM_KC / 16), col = (c % (LMM_KC / 16)) * 16;
            const int k = p * LMM_KC + col;
            v4i v = {0, 0, 0, 0};
            if (c < XCH && row < nb && k < n) v = *reinterpret_cast<const v4i *>(xq + (size_t)(b0 + row) * n + k);
            xr[j] = v;
        }
    };
    auto stage_x = [&](const v4i (&xr)[XPT], int buf) {
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            const int c = tid + j * 64 * LMM_WAVES;
            if (c < XCH) {
                const int row = c / (LMM_KC / 16), col = (c % (LMM_KC / 16)) * 16;
                *reinterpret_cast<v4i *>(&xs[buf][row * LMM_KC + col]) = xr[j];
            }
        }
    };

    for (int t0 = vlo; t0 < vhi; t0 += LMM_TILE_V) {
        const int v = t0 + 16 * wv + r16;  // this lane's w row (B operand column)
        const bool vok = v < vhi;
        const int8_t *wrow = w + (size_t)(vok ? v : 0) * n;
        auto fetch_w = [&](v4i (&f)[4], int p) {
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                const int k = p * LMM_KC + 64 * s4 + 16 * g;
                f[s4] = (vok && k < n) ? __builtin_nontemporal_load(reinterpret_cast<const v4i *>(wrow + k))
                                       : v4i{0, 0, 0, 0};
            }
        };
        v4i acc[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = v4i{0, 0, 0, 0};
        v4i w0[4], w1[4], w2[4];
        v4i xr[XPT];
        fetch_x(xr, 0);
        fetch_w(w0, 0);
        fetch_w(w1, 1);
        __syncthreads();  // the previous tile is done with both stage buffers
        stage_x(xr, 0);
        if (npass > 1) fetch_x(xr, 1);
        for (int p = 0; p < npass; ++p) {
            fetch_w(w2, p + 2);
            __syncthreads();  // stage p is in; stage p+1's buffer is free
            if (p + 1 < npass) {
                stage_x(xr, (p + 1) & 1);
                if (p + 2 < npass) fetch_x(xr, p + 2);
            }
            const int8_t *xb = xs[p & 1];
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const v4i a = *reinterpret_cast<const v4i *>(xb + (mt * 16 + r16) * LMM_KC + 64 * s4 + 16 * g);
                    acc[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, w0[s4], acc[mt], 0, 0, 0);
                }
            }
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                w0[s4] = w1[s4];
                w1[s4] = w2[s4];
            }
        }
        if (vok) {
            const float swv = sw[v];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int bb = mt * 16 + 4 * g + i;
                    if (bb < nb) logits[(size_t)(b0 + bb) * ld + v] = (sx[b0 + bb] * swv) * (float)acc[mt][i];
                }
        }
    }
}

// Int8 LM head over the packed weight layout (lal_gpu_pack_q8): block (T, c)
// = 1024 bytes holding w[16T + l%16][64c + 16(l/16) + j] at byte 16 l + j, the
// B operand of one v_mfma_i32_16x16x64_i8 as its 64 lanes load it, so every
// wave streams its 16 vocab rows as one contiguous run (n_pad bytes per row,
// 1 KB per load instruction).  Same arithmetic and A/C layouts as
// lm_head_mfma_kernel; a workgroup's tiles of 16 rows (one per wave at a time)
// and their passes of 256 k-bytes form one flat sequence of steps with two
// steps of w in flight across tile boundaries; the activations of a step are
// staged in LDS one step ahead, their global loads issued before the w loads
// of the same step (loads complete in issue order).  Batch rows 1..64.
template <int MT, int PD>
__global__ __launch_bounds__(64 * LMM_WAVES) void lm_head_packed_kernel(const int8_t *xq, const float *sx, int n,
                                                                        const int8_t *wpk, const float *sw, int V,
                                                                        float *logits, int ld, int b0, int nb)
{
    __shared__ __align__(16) int8_t xs[2][MT * 16 * LMM_KC];
    // a finished tile (MT*16 rows x 16 vocab, row-major) on its way out
    __shared__ __align__(16) float ot[MT > 1 ? LMM_WAVES : 1][MT > 1 ? MT * 256 : 4];
    constexpr int XCH = MT * 16 * (LMM_KC / 16);
    constexpr int XPT = (XCH + 64 * LMM_WAVES - 1) / (64 * LMM_WAVES);
    const int wv = wave_id(), lane = lane_id(), tid = threadIdx.x;
    const int g = lane >> 4, r16 = lane & 15;
    const int npass = (n + LMM_KC - 1) / LMM_KC;
    const int nc64 = (n + 63) / 64;           // 1 KB blocks per 16-row tile
    const int ntile = (V + 15) / 16;
    // this workgroup's tiles: [tlo, thi); wave wv takes tlo + wv, tlo + wv + 4, ...
    const int tlo = (int)(((long long)ntile * blockIdx.x) / gridDim.x);
    const int thi = (int)(((long long)ntile * (blockIdx.x + 1)) / gridDim.x);
    const int nround = (thi - tlo + LMM_WAVES - 1) / LMM_WAVES;
    const int nstep = nround * npass;
    if (nstep == 0) return;

    auto fetch_x = [&](v4i (&xr)[XPT], int p) {
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            const int c = tid + j * 64 * LMM_WAVES;
            const int row = c / (LMM_KC / 16), col = (c % (LMM_KC / 16)) * 16;
            const int k = p * LMM_KC + col;
            v4i v = {0, 0, 0, 0};
            if (c < XCH && row < nb && k < n) v = *reinterpret_cast<const v4i *>(xq + (size_t)(b0 + row) * n + k);
            xr[j] = v;
        }
    };
    // staged in A-operand order: the 16 bytes lane l = 16 g + r of
    // wave-instruction (mt, s4) reads sit in that instruction's 1 KB block at
    // slot 16 g + ((r + g + 4 s4) & 15).  The rotation keeps both sides free
    // of bank conflicts: any 8 consecutive chunks of one activation row
    // (g + 4 s4 = 0..7 or 8..15) land in 8 different 16-byte groups of a
    // 128-byte bank line, and the lanes of a read pass read consecutive
    // slots.
    auto stage_x = [&](const v4i (&xr)[XPT], int buf) {
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            const int c = tid + j * 64 * LMM_WAVES;
            if (c < XCH) {
                const int row = c / (LMM_KC / 16), c16 = c % (LMM_KC / 16);
                const int gg = c16 & 3, s4 = c16 >> 2;
                const int slot = gg * 16 + (((row & 15) + gg + 4 * s4) & 15);
                const int dst = (((row >> 4) * 4 + s4) * 64 + slot) * 16;
                *reinterpret_cast<v4i *>(&xs[buf][dst]) = xr[j];
            }
        }
    };
    // w of (round r, pass p): this wave's tile, blocks 4p .. 4p+3
    auto fetch_w = [&](v4i (&f)[4], int r, int p) {
        const int T = tlo + r * LMM_WAVES + wv;
        const bool ok = r < nround && T < thi;
        const v4i *base = reinterpret_cast<const v4i *>(wpk + ((size_t)(ok ? T : 0) * nc64) * 1024) + lane;
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
            const int c = 4 * p + s4;
            f[s4] = (ok && c < nc64) ? __builtin_nontemporal_load(base + (size_t)c * 64) : v4i{0, 0, 0, 0};
        }
    };

    v4i acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = v4i{0, 0, 0, 0};
    // the scales of this lane's batch rows (MT > 1), loaded once
    float sxr[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int bb = mt * 16 + 4 * g + i;
            sxr[mt][i] = (MT > 1 && bb < nb) ? sx[b0 + bb] : 0.0f;
        }
    const bool vec_out = ((ld & 3) == 0) && ((((uintptr_t)logits) & 15) == 0);
    v4i w0[4], w1[4], w2[4], w3[4];
    v4i xr[XPT];
    fetch_x(xr, 0);
    stage_x(xr, 0);
    fetch_x(xr, 1 % npass);  // activations of step 1, ahead of every w load
    // w of the first PD steps; (rw, pw) then holds the position of step PD
    int rw = 0, pw = 0;
    auto advance = [&]() {
        if (++pw == npass) { pw = 0; ++rw; }
    };
    fetch_w(w0, rw, pw);
    advance();
    fetch_w(w1, rw, pw);
    advance();
    if (PD == 3) {
        fetch_w(w2, rw, pw);
        advance();
    }
    int r = 0, p = 0;                                        // position of step s
    // one step: compute on wc (step s), load step s+PD into wn; the PD + 1
    // register sets rotate by unrolling, never by copies (a copy of a register
    // still being loaded would wait for that load)
    auto step = [&](int s, v4i (&wc)[4], v4i (&wn)[4]) {
        __syncthreads();  // step s's activations are in; the other buffer is free
        if (s + 1 < nstep) {
            stage_x(xr, (s + 1) & 1);
            if (s + 2 < nstep) fetch_x(xr, (s + 2) % npass);  // activations of step s+2
        }
        fetch_w(wn, rw, pw);
        advance();
        const int8_t *xb = xs[s & 1];
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
            const int slot = g * 16 + ((r16 + g + 4 * s4) & 15);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const v4i a = *reinterpret_cast<const v4i *>(xb + ((mt * 4 + s4) * 64 + slot) * 16);
                acc[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, wc[s4], acc[mt], 0, 0, 0);
            }
        }
        if (++p == npass) {  // the tile's dot products are complete
            const int T = tlo + r * LMM_WAVES + wv;
            const int v = 16 * T + r16;
            if (MT == 1 && T < thi && v < V) {
                const float swv = sw[v];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int bb = 4 * g + i;
                    if (bb < nb) logits[(size_t)(b0 + bb) * ld + v] = (sx[b0 + bb] * swv) * (float)acc[0][i];
                }
            } else if (MT > 1 && T < thi) {
                // through LDS, so that lane l stores float4 f = 64 q + l of the
                // tile (row f/4, vocab 16T + 4(f%4) ..), MT 16-byte stores per
                // lane instead of 4 MT scattered ones
                const float swv = (v < V) ? sw[v] : 0.0f;
                float *o = ot[MT > 1 ? wv : 0];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        o[(mt * 16 + 4 * g + i) * 16 + r16] = (sxr[mt][i] * swv) * (float)acc[mt][i];
                wave_sync();
#pragma unroll
                for (int q = 0; q < MT; ++q) {
                    const int f = q * 64 + lane, row = f >> 2, v0 = 16 * T + 4 * (f & 3);
                    const f32x4 val = *reinterpret_cast<const f32x4 *>(o + row * 16 + 4 * (f & 3));
                    if (row < nb) {
                        float *dst = logits + (size_t)(b0 + row) * ld + v0;
                        if (vec_out && v0 + 3 < V) {
                            *reinterpret_cast<f32x4 *>(dst) = val;
                        } else {
#pragma unroll
                            for (int c = 0; c < 4; ++c)
                                if (v0 + c < V) dst[c] = val[c];
                        }
                    }
                }
                wave_sync();  // the tile buffer is read before the next tile writes it
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[mt] = v4i{0, 0, 0, 0};
            p = 0;
            ++r;
        }
    };
    if (PD == 2) {
        for (int s = 0; s < nstep; s += 3) {
            step(s, w0, w2);
            if (s + 1 < nstep) step(s + 1, w1, w0);
            if (s + 2 < nstep) step(s + 2, w2, w1);
        }
    } else {
        for (int s = 0; s < nstep; s += 4) {
            step(s, w0, w3);
            if (s + 1 < nstep) step(s + 1, w1, w0);
            if (s + 2 < nstep) step(s + 2, w2, w1);
            if (s + 3 < nstep) step(s + 3, w3, w2);
        }
    }
}

// Int8 LM head over the packed layout for 33..64 batch rows with the
// activations resident in LDS.  k is split into two halves that the same
// workgroup (8 waves, one per CU) runs one after the other: half h of the
// batch's activations (MT*16 rows x at most 2 KB) is staged in LDS in
// A-operand order (the slot rotation of lm_head_packed_kernel), every wave
// streams W for its tiles with three steps in flight and no barrier per step,
// and it keeps each tile's first-half int32 sums in registers (at most
// LMK_MAXT tiles per wave) until its second pass over the tile adds the rest
// (integer sums are exact in any order).  W is read once and the activations
// twice per workgroup, instead of once per step.  Same arithmetic as
// lm_head_packed_kernel: logits = (sx*sw)*(float)dot.
//
// Dynamic LDS (lmk_lds_bytes): xs [4*P0 k-blocks][MT][64 slots][16 B], then
// per wave one finished tile (MT*16 rows x 16 floats), then the batch rows'
// sx and the workgroup's tiles' sw.
constexpr int LMK_WAVES = 8;
constexpr int LMK_MAXT = 5;  // tiles per wave (the host checks the workgroups' share)
constexpr int LMK_SWS = LMK_MAXT * LMK_WAVES * 16;
constexpr int LMK_XPT = 16;  // staged 16-byte chunks per thread: 64 rows x 8 passes x 256 B / 512 threads

__host__ __device__ constexpr size_t lmk_lds_bytes(int mt, int P0)
{
    return (size_t)4 * P0 * mt * 1024 + (size_t)LMK_WAVES * mt * 1024 + 64 * 4 + LMK_SWS * 4;
}

template <int MT>
__global__ __launch_bounds__(64 * LMK_WAVES) void lm_head_ksplit_kernel(const int8_t *xq, const float *sx, int n,
                                                                         const int8_t *wpk, const float *sw, int V,
                                                                         float *logits, int ld, int b0, int nb)
{
    extern __shared__ __align__(16) int8_t lmk_smem[];
    const int wv = wave_id(), lane = lane_id(), tid = threadIdx.x;
    const int g = lane >> 4, r16 = lane & 15;
    const int nc64 = (n + 63) / 64;
    const int npass = (nc64 + 3) / 4;
    const int P0 = (npass + 1) / 2;  // passes of the first half (the second has npass - P0 <= P0)
    int8_t *xs = lmk_smem;
    float *o = reinterpret_cast<float *>(lmk_smem + (size_t)4 * P0 * MT * 1024) + wv * MT * 256;
    float *sxs = reinterpret_cast<float *>(lmk_smem + (size_t)4 * P0 * MT * 1024 + LMK_WAVES * MT * 1024);
    float *sws = sxs + 64;
    const int ntile = (V + 15) / 16;
    const int tlo = (int)(((long long)ntile * blockIdx.x) / gridDim.x);
    const int thi = (int)(((long long)ntile * (blockIdx.x + 1)) / gridDim.x);
    const int ntile_w = (tlo + wv < thi) ? (thi - tlo - wv + LMK_WAVES - 1) / LMK_WAVES : 0;

    // the scales in LDS: the batch rows' sx, the workgroup's tiles' sw (read
    // where a tile is finished, not carried in registers)
    if (tid < 64) sxs[tid] = (tid < nb) ? sx[b0 + tid] : 0.0f;
    for (int i = tid; i < (thi - tlo) * 16; i += 64 * LMK_WAVES) {
        const int v = 16 * tlo + i;
        sws[i] = (v < V) ? sw[v] : 0.0f;
    }
    const bool vec_out = ((ld & 3) == 0) && ((((uintptr_t)logits) & 15) == 0);
    v4i saved[LMK_MAXT][MT];  // first-half sums of the wave's tiles
#pragma unroll
    for (int t = 0; t < LMK_MAXT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) saved[t][mt] = v4i{0, 0, 0, 0};

    for (int h = 0; h < 2; ++h) {
        const int pb = h ? P0 : 0;           // first pass of the half
        const int ph = h ? npass - P0 : P0;  // passes of the half
        // w of (round r, pass p of the half): this wave's tile, its blocks
        // 4 (pb + p) .. +3, every load issued (clamped; products past n meet
        // zero activations, padding steps are never stored)
        auto fetch_w = [&](v4i (&f)[4], int r, int p) {
            // a step past the wave's tiles reads again the blocks of its last
            // step of the half (just read: a cache hit)
            const bool ok = r < ntile_w;
            const int T = min(tlo + (ok ? r : max(ntile_w, 1) - 1) * LMK_WAVES + wv, ntile - 1);
            const int pc = ok ? p : ph - 1;
            const v4i *base = reinterpret_cast<const v4i *>(wpk + ((size_t)T * nc64) * 1024) + lane;
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                const int c = min(4 * (pb + pc) + s4, nc64 - 1);
                f[s4] = __builtin_nontemporal_load(base + (size_t)c * 64);
            }
        };
        // stage half h: chunk c = (row, c16), 16 bytes at k = 256 pb + 16 c16.
        // All of a thread's chunks are loaded at once (every load issued, at
        // a clamped address), then the first three steps' W, then the chunks
        // go to LDS: one round trip for the staging, overlapped with W.
        const int cph = 16 * ph;  // 16-byte chunks per row in the half
        v4i xr[LMK_XPT];
#pragma unroll
        for (int j = 0; j < LMK_XPT; ++j) {
            const int c = tid + j * 64 * LMK_WAVES;
            const int row = c / cph, k = 256 * pb + 16 * (c - row * cph);
            const bool in = c < MT * 16 * cph && row < nb && k < n;
            const v4i v = *reinterpret_cast<const v4i *>(xq + (in ? (size_t)(b0 + row) * n + k : 0));
            xr[j] = in ? v : v4i{0, 0, 0, 0};
        }
        __builtin_amdgcn_sched_barrier(0);
        v4i w0[4], w1[4], w2[4], w3[4];
        int rw = 0, pw = 0;
        auto advance = [&]() {
            if (++pw == ph) { pw = 0; ++rw; }
        };
        // issued in step order (the scheduler would otherwise reorder them,
        // and the loop's first wait would then cover every load in flight)
        fetch_w(w0, rw, pw);
        advance();
        __builtin_amdgcn_sched_barrier(0);
        fetch_w(w1, rw, pw);
        advance();
        __builtin_amdgcn_sched_barrier(0);
        fetch_w(w2, rw, pw);
        advance();
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();  // the previous half's readers are done
#pragma unroll
        for (int j = 0; j < LMK_XPT; ++j) {
            const int c = tid + j * 64 * LMK_WAVES;
            if (c < MT * 16 * cph) {
                const int row = c / cph, c16 = c - row * cph;
                const int gg = c16 & 3, kb = c16 >> 2;
                const int slot = gg * 16 + (((row & 15) + gg + 4 * (kb & 3)) & 15);
                *reinterpret_cast<v4i *>(&xs[((kb * MT + (row >> 4)) * 64 + slot) * 16]) = xr[j];
            }
        }
        __syncthreads();
        if (ntile_w == 0) continue;

        v4i acc[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = h ? saved[0][mt] : v4i{0, 0, 0, 0};
        int r = 0, p = 0;
        // a tile whose second half ended in this trip of four steps waits in
        // LDS (scaled) and is stored at the trip's end (ph >= 4: at most one
        // per trip), so that the unrolled steps make no global access but
        // their W loads and the compiler's wait counts see every load in
        // flight
        int r_c = 0;
        bool pend = false;
        auto step = [&](v4i (&wc)[4], v4i (&wn)[4]) __attribute__((always_inline)) {
            fetch_w(wn, rw, pw);
            advance();
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                const int slot = g * 16 + ((r16 + g + 4 * s4) & 15);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const v4i a = *reinterpret_cast<const v4i *>(xs + (((4 * p + s4) * MT + mt) * 64 + slot) * 16);
                    acc[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, wc[s4], acc[mt], 0, 0, 0);
                }
            }
            if (++p == ph) {  // this half of the tile is done
                if (h == 0) {
#pragma unroll
                    for (int t = 0; t < LMK_MAXT; ++t)
                        if (t == r)
#pragma unroll
                            for (int mt = 0; mt < MT; ++mt) saved[t][mt] = acc[mt];
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[mt] = v4i{0, 0, 0, 0};
                } else {
                    const float swv = sws[(r * LMK_WAVES + wv) * 16 + r16];
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const f32x4 s4v = *reinterpret_cast<const f32x4 *>(sxs + mt * 16 + 4 * g);
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            o[(mt * 16 + 4 * g + i) * 16 + r16] = (s4v[i] * swv) * (float)acc[mt][i];
                    }
                    r_c = r;
                    pend = true;
                    // the next tile starts from its first-half sums
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[mt] = v4i{0, 0, 0, 0};
#pragma unroll
                    for (int t = 1; t < LMK_MAXT; ++t)
                        if (t == r + 1)
#pragma unroll
                            for (int mt = 0; mt < MT; ++mt) acc[mt] = saved[t][mt];
                }
                ++r;
                p = 0;
            }
        };
        // tile r_c from LDS: lane l stores row 16 mt + l/4, vocab 16T +
        // 4(l%4) .. +3 (one 16-byte store per 16-row block)
        auto store_tile = [&]() __attribute__((always_inline)) {
            const int T = tlo + r_c * LMK_WAVES + wv;
            wave_sync();
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int R = mt * 16 + (lane >> 2), v0 = 16 * T + 4 * (lane & 3);
                const f32x4 val = *reinterpret_cast<const f32x4 *>(o + (mt * 16 + (lane >> 2)) * 16 + 4 * (lane & 3));
                if (R < nb && T < thi) {
                    float *dst = logits + (size_t)(b0 + R) * ld + v0;
                    if (vec_out && v0 + 3 < V) {
                        *reinterpret_cast<f32x4 *>(dst) = val;
                    } else {
#pragma unroll
                        for (int c = 0; c < 4; ++c)
                            if (v0 + c < V) dst[c] = val[c];
                    }
                }
            }
            wave_sync();  // read before the next tile overwrites it
        };
        const int nstep_w = ntile_w * ph;
        for (int s = 0; s < nstep_w; s += 4) {
            step(w0, w3);
            step(w1, w0);
            step(w2, w1);
            step(w3, w2);
            if (pend) {
                store_tile();
                pend = false;
            }
        }
    }
}

// Startup weight quantizer (runtime/lal_q8_kernel.h:357-372,
// lal_quantize_q8_per_row): per row, scale = max|w| / 127 (at least 1e-8),
// q = lroundf(w * (1/scale)) clamped to [-127, 127] (round half away from
// zero).  One workgroup per row; the maximum is order-free.
__global__ __launch_bounds__(256) void quantize_w_kernel(const float *w, int n, int8_t *q, float *scale)
{
    __shared__ float red[4];
    const int j = blockIdx.x;
    const float *r = w + (size_t)j * n;
    float m = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) m = fmaxf(m, fabsf(r[i]));
    m = wave_max(m);
    if (lane_id() == 0) red[wave_id()] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float s = m / 127.0f;
    if (s < 1e-8f) s = 1e-8f;
    const float inv = 1.0f / s;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float t = r[i] * inv;
        int v = (int)roundf(t);
        v = min(127, max(-127, v));
        q[(size_t)j * n + i] = (int8_t)v;
    }
    if (threadIdx.x == 0) scale[j] = s;
}

// Up to 16 batch rows with n <= LMX_MAXN: the activations of every pass stay
// in LDS for the whole launch (staged once, in A-operand order with the slot
// rotation of lm_head_packed_kernel, block kb per 64 k-bytes), so each wave
// streams its tiles' W with three steps in flight and no barrier per step.
// Same arithmetic as lm_head_packed_kernel<1, PD>.
//
// With CAND the tiles also keep, per batch row, the logits that can reach the
// row's top-k pool, for the sampler's list mode.  The bound: every wave's
// first tile is a fixed sample of the vocabulary (ns ids in all); a
// workgroup's per-row maximum over its four first tiles goes by atomicMax into
// slot blockIdx % 64 of the row, and a wave's bound is the ks-th largest slot,
// ks = ceil(lam + 6 sqrt(lam) + 6) with lam = k ns / V.  It exceeds the row's
// k-th largest only when ks of the row's top-k fall in the sample (each such
// value raises at most one slot), which for a random placement of the top-k
// is a Poisson tail of negligible mass.  Slots still empty when a wave reads
// them only lower its bound, and the final slots give a bound at least every
// wave's, so the sampler recomputes it from them and checks it (at least k
// list values at or above it), streaming the row otherwise.  A wave reads the
// slots after its second tile (or its only one) and filters its first tile's
// values then.  Passing values are staged per wave in LDS (CAND_ROW per row:
// about 200 of a row's values pass over some 2000 waves); the last wave of a
// workgroup to finish writes every wave's values out, one atomic per row
// reserving their place in sub-list (workgroup index % HSUB) of the row's
// list (one counter for all 512 workgroups serialised ~2000 atomics at the
// kernel's end).  A nan logit or a full stage or list flags the row.
constexpr int CAND_ROW = 8;
constexpr int LMX_MAXN = 4096;
struct HeadCand {
    int4 *hmeta;      // [row * HMETA_STRIDE] (-, -, -, flags: 1 full, 2 nan), then HSUB sub-list counts
    unsigned *hslots; // [row][64]
    float *lval;      // [row][hcap]
    int *lidx;
    int hcap;
    int ks;           // 1..64
};

// Candidate stage of lm_head_packed_xres_kernel<true>: per wave, per row
// CAND_ROW values, written out by the wave at its end.
struct CandStage {
    unsigned wgmax[16];  // per-row maximum key of the workgroup's first tiles
    int done0;           // waves past their first tile
    int done_end;        // waves past their last tile
    unsigned bkey[16];   // per-row bound key a wave of the workgroup took from the slots
    int bready;          // bkey is set
    int cnt[LMM_WAVES][16];  // staged values per row (may exceed CAND_ROW: full)
    float val[LMM_WAVES][16 * CAND_ROW];
    int id[LMM_WAVES][16 * CAND_ROW];
};

// stage this lane's value y of row `row` (vocab v) when it passes
__device__ __forceinline__ void cand_stage(CandStage &CS, int wv, int row, float y, int v, bool pass)
{
    if (!__ballot(pass)) return;
    if (pass) {
        const int pos = atomicAdd(&CS.cnt[wv][row], 1);
        if (pos < CAND_ROW) {
            CS.val[wv][row * CAND_ROW + pos] = y;
            CS.id[wv][row * CAND_ROW + pos] = v;
        }
    }
}

// In-kernel activation quantization (lal_quantize_x_int8, AVX2 build) of up
// to QX_ROWS rows: every workgroup quantizes the rows itself (they are small
// and stay in L2) instead of waiting for a separate launch; workgroup 0
// writes xq / sx out.
constexpr int QX_ROWS = 4;
struct HeadQuant {
    const float *x;  // [nb][n] fp32 (16-byte aligned), or null: xq / sx are inputs
    int8_t *xq;      // outputs of workgroup 0
    float *sx;
};

template <bool CAND>
__global__ __launch_bounds__(64 * LMM_WAVES) void lm_head_packed_xres_kernel(const int8_t *xq, const float *sx, int n,
                                                                             const int8_t *wpk, const float *sw,
                                                                             int V, float *logits, int ld, int b0,
                                                                             int nb, HeadCand C, HeadQuant HQ)
{
    __shared__ __align__(16) int8_t xs[16 * LMX_MAXN];
    __shared__ __align__(16) float ot[LMM_WAVES][16 * 16];  // a finished tile, row-major
    __shared__ CandStage CS;
    __shared__ QxShared QS;
    __shared__ float qsc[QX_ROWS][LMM_WAVES];  // per-row maxima, then scales
    const int wv = wave_id(), lane = lane_id(), tid = threadIdx.x;
    const int g = lane >> 4, r16 = lane & 15;
    if (CAND) {
        if (tid < 16) CS.wgmax[tid] = 0u;
        if (tid < 16 * LMM_WAVES) CS.cnt[tid >> 4][tid & 15] = 0;
        if (tid == 0) {
            CS.done0 = 0;
            CS.done_end = 0;
            CS.bready = 0;
        }
    }
    const int npass = (n + LMM_KC - 1) / LMM_KC;
    const int nc64 = (n + 63) / 64;  // 1 KB blocks per 16-row tile
    const int ntile = (V + 15) / 16;
    const int tlo = (int)(((long long)ntile * blockIdx.x) / gridDim.x);
    const int thi = (int)(((long long)ntile * (blockIdx.x + 1)) / gridDim.x);
    const int nround = (thi - tlo + LMM_WAVES - 1) / LMM_WAVES;
    const int nstep = nround * npass;

    // w of (round r, pass p): this wave's tile, blocks 4p .. 4p+3.  Every
    // load is issued (a wave past its tiles reads its last step's blocks
    // again, blocks past the row read its last one): with no branch around them the
    // compiler counts the loads in flight exactly and waits only for the step
    // it multiplies.  The extra products are exact zeros (the activations of
    // blocks past n are zero in LDS) or belong to tiles that are not stored.
    // this wave's tiles: tlo + wv + LMM_WAVES r for r < ntile_w
    const int ntile_w = (tlo + wv < thi) ? (thi - tlo - wv + LMM_WAVES - 1) / LMM_WAVES : 0;
    auto fetch_w = [&](v4i (&f)[4], int r, int p) {
        // a step past the wave's tiles reads again the blocks of its last
        // step (just read: a cache hit), not blocks read long ago
        const bool ok = r < ntile_w;
        const int Tc = min(tlo + (ok ? r : max(ntile_w, 1) - 1) * LMM_WAVES + wv, ntile - 1);
        const int pc = ok ? p : npass - 1;
        const v4i *base = reinterpret_cast<const v4i *>(wpk + ((size_t)Tc * nc64) * 1024) + lane;
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
            const int c = min(4 * pc + s4, nc64 - 1);
            f[s4] = __builtin_nontemporal_load(base + (size_t)c * 64);
        }
    };
    // the activations (chunk c = (row, c16), 16 bytes at k = 16 c16 of row
    // c / (4 nc64)) are loaded first, then the first three steps' W, then the
    // activations are stored to LDS (loads complete in issue order)
    constexpr int XR = 16 * (LMX_MAXN / 16) / (64 * LMM_WAVES);
    const int cpr = 4 * nc64;
    v4i xr[XR];
    // in-kernel quantization: chunk j of this thread as fp32 (16 values)
    constexpr int XQ = QX_ROWS * (LMX_MAXN / 16) / (64 * LMM_WAVES);
    f32x4 xf[XQ][4];
    if (CAND && HQ.x) {
#pragma unroll
        for (int j = 0; j < XQ; ++j) {
            const int c = tid + j * 64 * LMM_WAVES;
            const int row = c / cpr, k = 16 * (c - row * cpr);
            const bool in = row < nb && k < n;
            const f32x4 *src = reinterpret_cast<const f32x4 *>(HQ.x + (size_t)(b0 + (in ? row : 0)) * n + (in ? k : 0));
#pragma unroll
            for (int q = 0; q < 4; ++q) xf[j][q] = in ? src[q] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    } else {
#pragma unroll
        for (int j = 0; j < XR; ++j) {
            const int c = tid + j * 64 * LMM_WAVES;
            const int row = c / cpr, k = 16 * (c - row * cpr);
            v4i v = {0, 0, 0, 0};
            if (c < 16 * cpr && row < nb && k < n)
                v = *reinterpret_cast<const v4i *>(xq + (size_t)(b0 + row) * n + k);
            xr[j] = v;
        }
    }
    float qscl[QX_ROWS];  // the row scales of the in-kernel quantization
#pragma unroll
    for (int r = 0; r < QX_ROWS; ++r) qscl[r] = 0.0f;
    if (CAND && HQ.x) {
        // per-row max |x| and whether the row holds a nan or an infinity
        float m[QX_ROWS];
        bool bad[QX_ROWS];
#pragma unroll
        for (int r = 0; r < QX_ROWS; ++r) {
            m[r] = 0.0f;
            bad[r] = false;
        }
#pragma unroll
        for (int j = 0; j < XQ; ++j) {
            const int row = (tid + j * 64 * LMM_WAVES) / cpr;
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float a = fabsf(xf[j][q][e]);
#pragma unroll
                    for (int r = 0; r < QX_ROWS; ++r)
                        if (row == r) {
                            m[r] = fmaxf(m[r], a);
                            bad[r] = bad[r] || !(a <= 3.402823466e38f);
                        }
                }
        }
#pragma unroll
        for (int r = 0; r < QX_ROWS; ++r) {
            const float mw = wave_max(m[r]);
            const bool bw = __ballot(bad[r]) != 0ull;
            if (lane_id() == 0) qsc[r][wv] = bw ? -1.0f : mw;
        }
    }
    // W of the first three steps, after the activations' loads and maxima
    // (loads complete in issue order: waiting for the activations does not
    // wait for W)
    v4i w0[4], w1[4], w2[4], w3[4];
    int rw = 0, pw = 0;
    auto advance = [&]() {
        if (++pw == npass) { pw = 0; ++rw; }
    };
    fetch_w(w0, rw, pw);
    advance();
    fetch_w(w1, rw, pw);
    advance();
    fetch_w(w2, rw, pw);
    advance();
    if (CAND && HQ.x) {
        __syncthreads();
        float *scl = qscl;
#pragma unroll
        for (int r = 0; r < QX_ROWS; ++r) {
            float mm = 0.0f;
            bool bb = false;
#pragma unroll
            for (int ww = 0; ww < LMM_WAVES; ++ww) {
                bb = bb || qsc[r][ww] < 0.0f;
                mm = fmaxf(mm, qsc[r][ww]);
            }
            if (r < nb && bb) {
                // a nan or an infinity: the build's order decides the maximum
                scl[r] = qx_scale(HQ.x + (size_t)(b0 + r) * n, n, 0, QS);
            } else {
                scl[r] = mm / 127.0f;
                if (scl[r] < 1e-8f) scl[r] = 1e-8f;
            }
        }
        if (blockIdx.x == 0 && tid < nb && tid < QX_ROWS) {
#pragma unroll
            for (int r = 0; r < QX_ROWS; ++r)
                if (tid == r) HQ.sx[b0 + r] = scl[r];
        }
        // the quantized chunks (n is a multiple of 16: every value is in the
        // rounded prefix)
#pragma unroll
        for (int j = 0; j < XQ; ++j) {
            const int c = tid + j * 64 * LMM_WAVES;
            const int row = c / cpr, k = 16 * (c - row * cpr);
            float sc = 1.0f;
#pragma unroll
            for (int r = 0; r < QX_ROWS; ++r)
                if (row == r) sc = scl[r];
            const float inv = 1.0f / sc;
            int w4[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t u = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) u |= (uint32_t)(uint8_t)qx_value(xf[j][q][e], inv, true) << (8 * e);
                w4[q] = (int)u;
            }
            const v4i v = {w4[0], w4[1], w4[2], w4[3]};
            const bool in = row < nb && k < n;
            xr[j] = in ? v : v4i{0, 0, 0, 0};
            if (blockIdx.x == 0 && in) *reinterpret_cast<v4i *>(HQ.xq + (size_t)(b0 + row) * n + k) = v;
        }
#pragma unroll
        for (int j = XQ; j < XR; ++j) xr[j] = v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int j = 0; j < XR; ++j) {
        const int c = tid + j * 64 * LMM_WAVES;
        if (c < 16 * cpr) {
            const int row = c / cpr, c16 = c - row * cpr;
            const int gg = c16 & 3, kb = c16 >> 2;
            const int slot = gg * 16 + ((row + gg + 4 * (kb & 3)) & 15);
            *reinterpret_cast<v4i *>(&xs[(kb * 64 + slot) * 16]) = xr[j];
        }
    }
    // blocks of the last pass past the row: zero activations
    for (int i = tid; i < (4 * npass - nc64) * 64; i += 64 * LMM_WAVES)
        *reinterpret_cast<v4i *>(&xs[(nc64 * 64 + i) * 16]) = v4i{0, 0, 0, 0};
    __syncthreads();
    if (nstep == 0) return;

    // the scales of this lane's 4 batch rows, loaded once
    float sxr[4];
    if (CAND && HQ.x) {
        // the row scales as this workgroup computed them (rows < QX_ROWS:
        // only lanes of group 0 have rows)
#pragma unroll
        for (int i = 0; i < 4; ++i) sxr[i] = (g == 0 && i < nb) ? qscl[i] : 0.0f;
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) sxr[i] = (4 * g + i < nb) ? sx[b0 + 4 * g + i] : 0.0f;
    }
    const bool vec_out = ((ld & 3) == 0) && ((((uintptr_t)logits) & 15) == 0);
    // candidate state: the first tile's values, this lane's rows' bounds
    float y0[4] = {0.0f, 0.0f, 0.0f, 0.0f}, bnd[4] = {INFINITY, INFINITY, INFINITY, INFINITY};
    bool ok0[4] = {false, false, false, false};
    int v0 = 0;
    bool have_bnd = false;
    auto take_bound = [&]() __attribute__((always_inline)) {
        // the ks-th largest slot of every row, 16 rows side by side (bit by
        // bit, ballot counts), then the first tile's values against it.  The
        // first wave of the workgroup to get here reads the slots (a global
        // round trip that drains its W pipeline) and leaves the bounds in
        // LDS; a later wave takes them from there.  Any wave's bound is at
        // most the bound of the final slots (slots only grow), which the
        // sampler checks the list against.
        uint32_t K[16];
        const int ready = __builtin_amdgcn_readfirstlane(
            __hip_atomic_load(&CS.bready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP));
        if (ready) {
#pragma unroll
            for (int bb = 0; bb < 16; ++bb) K[bb] = (bb < nb) ? CS.bkey[bb] : 0u;
        } else {
            uint32_t sk[16];
#pragma unroll
            for (int bb = 0; bb < 16; ++bb) {
                sk[bb] = (bb < nb) ? __hip_atomic_load(&C.hslots[(size_t)(b0 + bb) * 64 + lane], __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT)
                                   : 0u;
                K[bb] = 0u;
            }
            // the top 16 bits of the keys only (sign, exponent, 7 mantissa
            // bits): K is then at most the exact ks-th largest key, a lower
            // bound that lets through a few more values at half the ballots
            // (16 rows x 32 bits cost a wave ~4 us)
#pragma unroll 1
            for (int bit = 31; bit >= 16; --bit) {
#pragma unroll
                for (int bb = 0; bb < 16; ++bb) {
                    if (bb >= nb) break;
                    const uint32_t cand = K[bb] | (1u << bit);
                    if (__popcll(__ballot(sk[bb] >= cand)) >= C.ks) K[bb] = cand;
                }
            }
            if (lane == 0) {
#pragma unroll
                for (int bb = 0; bb < 16; ++bb)
                    if (bb < nb) CS.bkey[bb] = K[bb];
                __hip_atomic_store(&CS.bready, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        }
#pragma unroll
        for (int bb = 0; bb < 16; ++bb) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (4 * g + i == bb) bnd[i] = K[bb] ? keyf(K[bb]) : -INFINITY;
        }
        have_bnd = true;
#pragma unroll
        for (int i = 0; i < 4; ++i) cand_stage(CS, wv, 4 * g + i, y0[i], v0, ok0[i] && y0[i] >= bnd[i]);
    };
    v4i acc_c = {0, 0, 0, 0};  // a finished tile waiting for cand_tile
    float sw_c = 0.0f;
    int t_c = 0, r_c = 0;
    bool pend = false;
    auto cand_tile = [&]() __attribute__((always_inline)) {
        const int v = 16 * t_c + r16;
        const float swv = (v < V) ? sw_c : 0.0f;
        float y[4];
        bool ok[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ok[i] = v < V && 4 * g + i < nb;
            y[i] = (sxr[i] * swv) * (float)acc_c[i];
        }
        if (__ballot((ok[0] && y[0] != y[0]) || (ok[1] && y[1] != y[1]) || (ok[2] && y[2] != y[2]) ||
                     (ok[3] && y[3] != y[3]))) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (ok[i] && y[i] != y[i]) atomicOr(&C.hmeta[(size_t)(b0 + 4 * g + i) * HMETA_STRIDE].w, 2);
        }
        if (r_c == 0) {
            // the sample: per-row maxima of the 16 lanes of a group, then of
            // the workgroup's waves in LDS; the last wave past its first tile
            // publishes them to the row's slot (one atomic per row)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t m = ok[i] ? fkey(y[i]) : 0u;
                m = max(m, (uint32_t)__shfl_xor((int)m, 1, 64));
                m = max(m, (uint32_t)__shfl_xor((int)m, 2, 64));
                m = max(m, (uint32_t)__shfl_xor((int)m, 4, 64));
                m = max(m, (uint32_t)__shfl_xor((int)m, 8, 64));
                if (r16 == 0 && 4 * g + i < nb && m) atomicMax(&CS.wgmax[4 * g + i], m);
                y0[i] = y[i];
                ok0[i] = ok[i];
            }
            v0 = v;
            int prev = 0;
            if (lane == 0) prev = atomicAdd(&CS.done0, 1);
            prev = __builtin_amdgcn_readfirstlane(prev);
            if (prev == min(LMM_WAVES, thi - tlo) - 1 && lane < nb) {
                const unsigned m = CS.wgmax[lane];
                if (m) atomicMax(&C.hslots[(size_t)(b0 + lane) * 64 + (blockIdx.x & 63)], m);
            }
        } else {
            if (!have_bnd) take_bound();
#pragma unroll
            for (int i = 0; i < 4; ++i) cand_stage(CS, wv, 4 * g + i, y[i], v, ok[i] && y[i] >= bnd[i]);
        }
        pend = false;
    };
    v4i acc = {0, 0, 0, 0};
    int r = 0, p = 0;  // position of step s
    // sw of this lane's vocab row in the current tile, loaded one step ahead
    // (unconditionally, like W)
    auto sw_of = [&](int rr) {
        return sw[min(16 * min(tlo + rr * LMM_WAVES + wv, ntile - 1) + r16, V - 1)];
    };
    float sw_cur = sw_of(0);
    auto step = [&](v4i (&wc)[4], v4i (&wn)[4]) __attribute__((always_inline)) {
        fetch_w(wn, rw, pw);  // step s + 3
        advance();
        const float sw_next = sw_of(r + (p + 1 == npass ? 1 : 0));
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
            const int slot = g * 16 + ((r16 + g + 4 * s4) & 15);
            const v4i a = *reinterpret_cast<const v4i *>(xs + ((4 * p + s4) * 64 + slot) * 16);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, wc[s4], acc, 0, 0, 0);
        }
        if (++p == npass) {  // the tile's dot products are complete
            const int T = tlo + r * LMM_WAVES + wv;
            if (T < thi && nb <= 4) {
                const int v = 16 * T + r16;
                if (v < V) {
                    const float swv = sw_cur;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int bb = 4 * g + i;
                        if (bb < nb) logits[(size_t)(b0 + bb) * ld + v] = (sxr[i] * swv) * (float)acc[i];
                    }
                }
            } else if (T < thi) {
                // lane (g, r16) holds rows 4g..4g+3 of vocab row 16T + r16; a
                // pass through LDS gives lane l row l/4, vocab 16T + 4(l%4) ..
                // +3, so that the tile leaves in one 16-byte store per lane
                // instead of four scattered ones (the store count, not the
                // bytes, costs at 5-16 rows)
                const int v = 16 * T + r16;
                const float swv = (v < V) ? sw_cur : 0.0f;
                float *o = ot[wv];
#pragma unroll
                for (int i = 0; i < 4; ++i) o[(4 * g + i) * 16 + r16] = (sxr[i] * swv) * (float)acc[i];
                wave_sync();
                const int R = lane >> 2, v0 = 16 * T + 4 * (lane & 3);
                const f32x4 val = *reinterpret_cast<const f32x4 *>(o + R * 16 + 4 * (lane & 3));
                if (R < nb) {
                    float *dst = logits + (size_t)(b0 + R) * ld + v0;
                    if (vec_out && v0 + 3 < V) {
                        *reinterpret_cast<f32x4 *>(dst) = val;
                    } else {
#pragma unroll
                        for (int c = 0; c < 4; ++c)
                            if (v0 + c < V) dst[c] = val[c];
                    }
                }
                wave_sync();  // the tile buffer is read before the next tile writes it
            }
            if (CAND && T < thi) {
                // handled after this group of four steps (a tile spans at
                // least four, so at most one is pending)
                acc_c = acc;
                sw_c = sw_cur;
                t_c = T;
                r_c = r;
                pend = true;
            }
            acc = v4i{0, 0, 0, 0};
            p = 0;
            ++r;
        }
        sw_cur = sw_next;
    };
    // four steps per trip with no branch between them (steps past the wave's
    // own belong to rounds past its tiles: computed, never stored), so that
    // the compiler's wait counts see every load of the trip; a wave stops
    // after its own tiles
    const int nstep_w = ntile_w * npass;
    for (int s = 0; s < nstep_w; s += 4) {
        step(w0, w3);
        step(w1, w0);
        step(w2, w1);
        step(w3, w2);
        if (CAND && pend) cand_tile();
    }
    // a wave with one tile reads the slots at its end
    if (CAND && !have_bnd && tlo + wv < thi) take_bound();
    if (CAND) {
        // the last wave of the workgroup to get here writes every wave's
        // staged values to sub-list (blockIdx % HSUB) of their rows: lane
        // l < nb reserves row l's places with one atomic (the waves' LDS
        // writes are ordered before their arrival by the release / acquire)
        int prev = 0;
        if (lane == 0)
            prev = __hip_atomic_fetch_add(&CS.done_end, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
        prev = __builtin_amdgcn_readfirstlane(prev);
        if (prev != LMM_WAVES - 1) return;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        int putw[LMM_WAVES];
        int tot = 0;
        bool over = false;
#pragma unroll
        for (int ww = 0; ww < LMM_WAVES; ++ww) {
            const int c = (lane < nb) ? CS.cnt[ww][lane] : 0;
            putw[ww] = min(c, CAND_ROW);
            tot += putw[ww];
            over = over || c > CAND_ROW;
        }
        const int sq = (int)(blockIdx.x % HSUB), subcap = C.hcap / HSUB;
        int base = 0;
        if (lane < nb && tot > 0) {
            int4 *hm = C.hmeta + (size_t)(b0 + lane) * HMETA_STRIDE;
            base = atomicAdd(&hm[1 + sq].x, tot);
            if (over || base + tot > subcap) atomicOr(&hm->w, 1);
        }
        for (int row = 0; row < nb; ++row) {
            const int tr = __builtin_amdgcn_readlane(tot, row), br = __builtin_amdgcn_readlane(base, row);
            for (int j = lane; j < tr; j += 64) {
                // entry j of the row: wave ww's staged value jj
                int ww = 0, jj = j;
#pragma unroll
                for (int q = 0; q < LMM_WAVES - 1; ++q) {
                    const int pq = __builtin_amdgcn_readlane(putw[q], row);
                    if (ww == q && jj >= pq) {
                        jj -= pq;
                        ww = q + 1;
                    }
                }
                if (br + j < subcap) {
                    const size_t o = (size_t)(b0 + row) * C.hcap + (size_t)sq * subcap + br + j;
                    C.lval[o] = CS.val[ww][row * CAND_ROW + jj];
                    C.lidx[o] = CS.id[ww][row * CAND_ROW + jj];
                }
            }
        }
    }
}

// Row-major int8 [V][n] -> packed layout (one thread per 16 bytes).
__global__ __launch_bounds__(256) void pack_q8_kernel(const int8_t *w, int V, int n, int8_t *wpk)
{
    const int nc64 = (n + 63) / 64;
    const size_t nblk = (size_t)((V + 15) / 16) * nc64;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;  // 16-byte unit
    if (i >= nblk * 64) return;
    const size_t blk = i >> 6;
    const int l = (int)(i & 63);
    const int T = (int)(blk / nc64), c = (int)(blk % nc64);
    const int v = 16 * T + (l & 15), k0 = 64 * c + 16 * (l >> 4);
    v4i out = {0, 0, 0, 0};
    if (v < V) {
        if (((n & 15) == 0) && k0 + 16 <= n) {
            out = *reinterpret_cast<const v4i *>(w + (size_t)v * n + k0);
        } else {
            int8_t b[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) b[j] = (k0 + j < n) ? w[(size_t)v * n + k0 + j] : (int8_t)0;
            out = *reinterpret_cast<const v4i *>(b);
        }
    }
    *reinterpret_cast<v4i *>(wpk + i * 16) = out;
}

// Rows whose length is not a multiple of 16 bytes: one wave per vocab row,
// byte loads, same exact int32 accumulation.
__global__ __launch_bounds__(256) void lm_head_scalar_kernel(const int8_t *xq, const float *sx, int n,
                                                             const int8_t *w, const float *sw, int V,
                                                             float *logits, int ld, int batch)
{
    const int v = blockIdx.x * 4 + wave_id();
    if (v >= V) return;
    const int8_t *wr = w + (size_t)v * n;
    for (int b = 0; b < batch; ++b) {
        int a = 0;
        for (int i = lane_id(); i < n; i += 64) a += (int)wr[i] * (int)xq[(size_t)b * n + i];
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) a += __shfl_xor(a, d, 64);
        if (lane_id() == 0) logits[(size_t)b * ld + v] = (sx[b] * sw[v]) * (float)a;
    }
}

// ---------------------------------------------------------------------------
// GPT-2 LM head, pass 2 (tools/server/gpt2_server.c:2155-2215): the R largest
// int8 logits of a row are re-scored in fp32.  The set is the one the
// reference's min-heap of R (index order, a value enters when the heap has
// room or it exceeds the root) keeps.  It is every value >= the R-th largest
// T (with multiplicity) unless values equal to T straddle the boundary: then
// which of them stay depends on the heap's history, and wave 0 replays the
// heap (a wave filters each 64 values against the root, one lane applies the
// pushes and root replacements in order).
// One workgroup of 1024 threads per row; the row (at most RR_VPT * 1024
// values) is held in registers, T is found bit by bit with block-wide counts
// from the highest bit where the row's largest and smallest keys differ.
// ---------------------------------------------------------------------------
constexpr int RERANK_MAX = 512;
constexpr int RERANK_MAXN = 8192;  // hidden size staged in LDS
constexpr int RR_WG = 1024;
constexpr int RR_WAVES = RR_WG / 64;
constexpr int RR_VPT = 64;         // row values per thread: vocab <= 65536

constexpr int RR_CAP = 1024;       // gathered keys for the exact search

struct RerankSmem {
    float hv[RERANK_MAX];
    int hi[RERANK_MAX];
    int red[2][RR_WAVES];
    unsigned redk[2][RR_WAVES];
    unsigned gk[RR_WG > RR_CAP ? RR_WG : RR_CAP];  // threads' largest keys, then the gathered keys
    int gi[RR_CAP];       // ... and their ids
    unsigned bound;
    int flag;
};

__device__ __forceinline__ int rr_block_sum(RerankSmem &S, int v, int slot)
{
    v = wave_sum(v);
    if (lane_id() == 0) S.red[slot][wave_id()] = v;
    __syncthreads();
    int t = 0;
#pragma unroll
    for (int w = 0; w < RR_WAVES; ++w) t += S.red[slot][w];
    return t;
}

// k-th largest of the keys q[0..NQ) held by one wave's lanes (0 = none), bit
// by bit from the top bit where lo and hi differ (lo <= every candidate <= hi):
// the largest K with at least k keys >= K.  Per-lane counts summed across the
// wave; wave-synchronous.
template <int NQ>
__device__ __forceinline__ uint32_t rr_wave_kth(const uint32_t (&q)[NQ], int k, uint32_t lo, uint32_t hi)
{
    if (lo >= hi) return hi;
    const int top = 31 - __builtin_clz(lo ^ hi);
    uint32_t K = (top == 31) ? 0u : (hi & ~((2u << top) - 1u));
    for (int bit = top; bit >= 0; --bit) {
        const uint32_t cand = K | (1u << bit);
        // per-lane count as a pairwise tree (short dependency chains)
        int t[NQ];
#pragma unroll
        for (int i = 0; i < NQ; ++i) t[i] = (q[i] >= cand) ? 1 : 0;
#pragma unroll
        for (int h = 1; h < NQ; h *= 2)
#pragma unroll
            for (int i = 0; i + h < NQ; i += 2 * h) t[i] += t[i + h];
        if (wave_sum(t[0]) >= k) K = cand;
    }
    return K;
}

__global__ __launch_bounds__(RR_WG) void rerank_select_kernel(int V, int R, const float *logits, int ld, int *out_ids)
{
    __shared__ RerankSmem S;
    const int b = blockIdx.x, tid = threadIdx.x, lane = lane_id(), w = wave_id();
    const float *row = logits + (size_t)b * ld;
    const int r_eff = min(R, V);
    // the row's keys (0 = past the row)
    uint32_t key[RR_VPT];
    uint32_t kx = 0u, kn = 0xFFFFFFFFu;
    float val[RR_VPT];
#pragma unroll
    for (int j = 0; j < RR_VPT; ++j) val[j] = row[min(tid + RR_WG * j, V - 1)];  // one burst of loads
#pragma unroll
    for (int j = 0; j < RR_VPT; ++j) {
        const bool in = tid + RR_WG * j < V;
        key[j] = in ? fkey(val[j]) : 0u;
        kx = max(kx, key[j]);
        kn = min(kn, in ? key[j] : 0xFFFFFFFFu);
    }
    S.gk[tid] = kx;  // this thread's largest key
    kx = wave_max_u(kx);
    kn = wave_min_u(kn);
    if (lane == 0) {
        S.redk[0][w] = kx;
        S.redk[1][w] = kn;
    }
    __syncthreads();
    kx = 0u;
    kn = 0xFFFFFFFFu;
#pragma unroll
    for (int ww = 0; ww < RR_WAVES; ++ww) {
        kx = max(kx, S.redk[0][ww]);
        kn = min(kn, S.redk[1][ww]);
    }
    // A lower bound L of T: the r_eff-th largest of the threads' largest keys
    // (r_eff distinct row values reach it); the keys >= L then hold the pool.
    if (w == 0) {
        uint32_t L = 0u;
        if (V > RR_CAP) {
            uint32_t q[RR_WG / 64], qx = 0u, qn = 0xFFFFFFFFu;
#pragma unroll
            for (int i = 0; i < RR_WG / 64; ++i) {
                q[i] = S.gk[lane + 64 * i];
                qx = max(qx, q[i]);
                qn = min(qn, q[i]);
            }
            // every thread holds a row value here (V > RR_CAP >= RR_WG), so
            // the answer lies within the maxima's own range
            L = rr_wave_kth<RR_WG / 64>(q, r_eff, wave_min_u(qn), wave_max_u(qx));
        }
        if (lane == 0) S.bound = L;
    }
    __syncthreads();
    const uint32_t L = S.bound;
    int mine = 0;
#pragma unroll
    for (int j = 0; j < RR_VPT; ++j) mine += (key[j] >= L && key[j] != 0u) ? 1 : 0;
    const int incl = wave_incl_scan(mine);
    if (lane == 63) S.red[0][w] = incl;
    __syncthreads();
    int ng = 0, off = incl - mine;
#pragma unroll
    for (int ww = 0; ww < RR_WAVES; ++ww) {
        ng += S.red[0][ww];
        off += (ww < w) ? S.red[0][ww] : 0;
    }
    uint32_t K;
    bool replay;
    if (ng >= r_eff && ng <= RR_CAP) {
        // gather the keys >= L (they hold the top r_eff), exact search by wave 0
#pragma unroll
        for (int j = 0; j < RR_VPT; ++j)
            if (key[j] >= L && key[j] != 0u) {
                S.gk[off] = key[j];
                S.gi[off] = tid + RR_WG * j;
                off++;
            }
        __syncthreads();
        if (w == 0) {
            uint32_t q[RR_CAP / 64];
#pragma unroll
            for (int i = 0; i < RR_CAP / 64; ++i) q[i] = (lane + 64 * i < ng) ? S.gk[lane + 64 * i] : 0u;
            const uint32_t Kw = rr_wave_kth<RR_CAP / 64>(q, r_eff, max(L, kn), kx);
            int nge = 0;
#pragma unroll
            for (int i = 0; i < RR_CAP / 64; ++i) nge += __popcll(__ballot(q[i] >= Kw && q[i] != 0u));
            if (lane == 0) {
                S.bound = Kw;
                S.flag = (nge != r_eff) ? 1 : 0;  // values equal to T straddle the boundary
            }
            if (nge == r_eff) {
                // every gathered key >= T, compacted in gather order
                int base = 0;
#pragma unroll
                for (int i = 0; i < RR_CAP / 64; ++i) {
                    const bool p = q[i] >= Kw && q[i] != 0u;
                    const unsigned long long m = __ballot(p);
                    if (p) S.hi[base + lanes_below(m)] = S.gi[lane + 64 * i];
                    base += __popcll(m);
                }
            }
        }
        __syncthreads();
        K = S.bound;
        replay = S.flag != 0;
    } else {
        // the bound failed or left too many: search the whole row
        K = kx;
        if (kn < kx) {
            const int top = 31 - __builtin_clz(kn ^ kx);
            K = (top == 31) ? 0u : (kx & ~((2u << top) - 1u));
            for (int bit = top, slot = 1; bit >= 0; --bit, slot ^= 1) {
                const uint32_t cand = K | (1u << bit);
                int c = 0;
#pragma unroll
                for (int j = 0; j < RR_VPT; ++j) c += (key[j] >= cand) ? 1 : 0;
                if (rr_block_sum(S, c, slot) >= r_eff) K = cand;
            }
        }
        int na = 0, ne = 0;
#pragma unroll
        for (int j = 0; j < RR_VPT; ++j) {
            na += (key[j] > K) ? 1 : 0;
            ne += (key[j] == K && key[j] != 0u) ? 1 : 0;
        }
        __syncthreads();
        const int n_above = rr_block_sum(S, na, 0);
        const int n_eq = rr_block_sum(S, ne, 1);
        replay = n_above + n_eq != r_eff;
        if (!replay) {
            int m2 = na + ne;
            const int inc2 = wave_incl_scan(m2);
            __syncthreads();
            if (lane == 63) S.red[0][w] = inc2;
            __syncthreads();
            int o2 = inc2 - m2;
            for (int ww = 0; ww < w; ++ww) o2 += S.red[0][ww];
#pragma unroll
            for (int j = 0; j < RR_VPT; ++j)
                if (key[j] >= K && key[j] != 0u) S.hi[o2++] = tid + RR_WG * j;
        }
    }
    if (replay && w == 0) {
        // the reference heap (gpt2_server.c:2165-2192), replayed in index
        // order: in each chunk of 64, the first value that acts on the
        // current heap (any while it fills, then above the root) is applied
        // by lane 0; values before it cannot act, as the heap is unchanged
        int size = 0;
        for (int base = 0; base < V; base += 64) {
            const int v = base + lane;
            const float x = (v < V) ? row[v] : 0.0f;
            unsigned long long todo = __ballot(v < V);
            while (todo) {
                const float root = (size < R) ? -INFINITY : S.hv[0];
                const unsigned long long m = __ballot(size < R || x > root) & todo;
                if (!m) break;
                const int l = (int)__builtin_ctzll(m);
                const float xv = readlane_f(x, l);
                if (lane == 0) {
                    if (size < R) {
                        int c = size;
                        S.hv[c] = xv;
                        S.hi[c] = base + l;
                        while (c > 0) {
                            const int pp = (c - 1) >> 1;
                            if (S.hv[pp] <= S.hv[c]) break;
                            const float tv = S.hv[pp]; S.hv[pp] = S.hv[c]; S.hv[c] = tv;
                            const int ti = S.hi[pp]; S.hi[pp] = S.hi[c]; S.hi[c] = ti;
                            c = pp;
                        }
                    } else {
                        S.hv[0] = xv;
                        S.hi[0] = base + l;
                        int pp = 0;
                        for (;;) {
                            const int lc = 2 * pp + 1, rc = 2 * pp + 2;
                            int sm = pp;
                            if (lc < size && S.hv[lc] < S.hv[sm]) sm = lc;
                            if (rc < size && S.hv[rc] < S.hv[sm]) sm = rc;
                            if (sm == pp) break;
                            const float tv = S.hv[pp]; S.hv[pp] = S.hv[sm]; S.hv[sm] = tv;
                            const int ti = S.hi[pp]; S.hi[pp] = S.hi[sm]; S.hi[sm] = ti;
                            pp = sm;
                        }
                    }
                }
                if (size < R) ++size;
                wave_sync();
                todo &= (l == 63) ? 0ull : (~0ull << (l + 1));
            }
        }
    }
    __syncthreads();
    for (int j = tid; j < r_eff; j += RR_WG) out_ids[(size_t)b * R + j] = S.hi[j];
}

// fp32 re-score (gpt2_server.c:2200-2213) of the kept ids, RR_PER of them per
// workgroup: their int8 rows are staged in LDS (one load burst), then lane c
// of a group of 8 runs the fused multiply-add chain over i = c mod 8 of
// w_row[i] = wq[i] * scale; the group's first lane sums the 8 chains in lane
// order and adds the tail one fused multiply-add at a time.
constexpr int RR_SCORE_WG = 512;
constexpr int RR_PER = RR_SCORE_WG / 8;       // candidates per workgroup
constexpr int RR_STAGE = 64 * 1024;           // staged row bytes
__global__ __launch_bounds__(RR_SCORE_WG) void rerank_score_kernel(const float *xs, int n, const int8_t *wq,
                                                                   const float *ws, int V, int R, float *logits,
                                                                   int ld, const int *ids)
{
    __shared__ float xsh[RERANK_MAXN];
    __shared__ __align__(16) int8_t rows[RR_STAGE];
    const int b = blockIdx.x, tid = threadIdx.x, lane = lane_id();
    const int r_eff = min(R, V);
    const int rs = (n + 4) & ~3;                        // staged row stride (bank spread)
    const int per = min(RR_PER, RR_STAGE / rs);         // candidates this workgroup holds
    const int j0 = blockIdx.y * per;
    const int cnt = min(per, r_eff - j0);
    if (cnt <= 0) return;
    const float *xr = xs + (size_t)b * n;
    for (int i = tid; i < n; i += RR_SCORE_WG) xsh[i] = xr[i];
    const int *idr = ids + (size_t)b * R + j0;
    if ((n & 15) == 0 && (((uintptr_t)wq) & 15) == 0) {
        const int c16 = n >> 4;
        for (int t = tid; t < cnt * c16; t += RR_SCORE_WG) {
            const int g = t / c16, c = t - g * c16;
            const int4 v4 = *reinterpret_cast<const int4 *>(wq + (size_t)idr[g] * n + 16 * c);
            int *d = reinterpret_cast<int *>(rows + g * rs + 16 * c);
            d[0] = v4.x; d[1] = v4.y; d[2] = v4.z; d[3] = v4.w;
        }
    } else {
        for (int t = tid; t < cnt * n; t += RR_SCORE_WG) {
            const int g = t / n, i = t - g * n;
            rows[g * rs + i] = wq[(size_t)idr[g] * n + i];
        }
    }
    __syncthreads();
    const int g = tid >> 3, c8 = tid & 7;
    const int n8 = n & ~7;
    float acc = 0.0f;
    float sc = 0.0f;
    int v = 0;
    if (g < cnt) {
        v = idr[g];
        sc = ws[v];
        const int8_t *wr = rows + g * rs;
        for (int i = c8; i < n8; i += 8) acc = fmaf(xsh[i], (float)wr[i] * sc, acc);
    }
    float part[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) part[c] = __shfl(acc, (lane & ~7) + c, 64);
    if (g < cnt && c8 == 0) {
        float sum = part[0];
#pragma unroll
        for (int c = 1; c < 8; ++c) sum = sum + part[c];
        const int8_t *wr = rows + g * rs;
        for (int i = n8; i < n; ++i) sum = fmaf(xsh[i], (float)wr[i] * sc, sum);
        logits[(size_t)b * ld + v] = sum;
    }
}

// ---------------------------------------------------------------------------
// synthetic workloads (benchmarks / tests)
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t mix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float u01(uint64_t h) { return (float)(h >> 40) * (1.0f / 16777216.0f); }

__device__ __forceinline__ float gauss(uint64_t h)
{
    const float u1 = ((float)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
    const float u2 = (float)((h >> 16) & 0xFFFFFF) * (1.0f / 16777216.0f);
    return sqrtf(-2.0f * logf(u1)) * cospif(2.0f * u2);
}

__global__ void synth_gauss_kernel(float *out, int V, int ld, uint64_t seed, float sigma,
                                   float offr, int nout, float outv)
{
    const int b = blockIdx.y;
    const uint64_t rs = mix64(seed ^ mix64((uint64_t)b + 0x1234567ull));
    const float off = offr != 0.0f ? (u01(mix64(rs ^ 0xABCDEFull)) * 2.0f - 1.0f) * offr : 0.0f;
    for (int v = blockIdx.x * blockDim.x + threadIdx.x; v < V; v += gridDim.x * blockDim.x) {
        float x = sigma * gauss(mix64(rs + (uint64_t)v)) + off;
        out[(size_t)b * ld + v] = x;
    }
    __syncthreads();
    if (blockIdx.x == 0 && (int)threadIdx.x < nout) {
        const int v = (int)(mix64(rs ^ (0x5151ull + threadIdx.x)) % (uint64_t)V);
        out[(size_t)b * ld + v] = outv;
    }
}

__global__ void synth_zipf_kernel(float *out, int V, int ld, uint64_t seed, float slope, float noise)
{
    const int b = blockIdx.y;
    const uint64_t rs = mix64(seed ^ mix64((uint64_t)b + 0x777ull));
    // rank(v) = (a*v + c) mod V + 1 with gcd(a, V) = 1 (a odd, not multiple of 3)
    uint64_t a = (mix64(rs) % (uint64_t)V) | 1ull;
    while ((V % 3 == 0 && a % 3 == 0) || (V % 7 == 0 && a % 7 == 0) || (V % 11 == 0 && a % 11 == 0) ||
           (V % 5 == 0 && a % 5 == 0) || (V % 13 == 0 && a % 13 == 0))
        a += 2;
    const uint64_t c = mix64(rs + 1) % (uint64_t)V;
    for (int v = blockIdx.x * blockDim.x + threadIdx.x; v < V; v += gridDim.x * blockDim.x) {
        const uint64_t rank = (a * (uint64_t)v + c) % (uint64_t)V + 1;
        const float x = -slope * logf((float)rank) + noise * gauss(mix64(rs + 77 + (uint64_t)v));
        out[(size_t)b * ld + v] = x;
    }
}

__global__ void synth_bits_kernel(uint32_t *out, int V, int wld, uint64_t seed, float p)
{
    const int b = blockIdx.y;
    const int nw = (V + 31) / 32;
    for (int w = blockIdx.x * blockDim.x + threadIdx.x; w < wld; w += gridDim.x * blockDim.x) {
        uint32_t bits = 0;
        if (w < nw) {
            for (int j = 0; j < 32; ++j) {
                const int v = 32 * w + j;
                if (v < V && u01(mix64(seed ^ mix64(((uint64_t)b << 32) + (uint64_t)v))) < p)
                    bits |= 1u << j;
            }
        }
        out[(size_t)b * wld + w] = bits;
    }
}

__global__ void synth_int8_kernel(int8_t *out, size_t n, uint64_t seed, int lo, int hi)
{
    const uint64_t span = (uint64_t)(hi - lo + 1);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = (int8_t)(lo + (int)(mix64(seed + i) % span));
}

__global__ void synth_uniform_kernel(float *out, size_t n, uint64_t seed, float lo, float hi)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = lo + (hi - lo) * u01(mix64(seed + i));
}

__global__ void synth_normal_kernel(float *out, size_t n, uint64_t seed, float sigma)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = sigma * gauss(mix64(seed + i));
}

// Plain streaming copy (16-byte loads and stores, grid-stride): the yardstick
// that HBM byte counters are scaled by.
__global__ __launch_bounds__(256) void copy_f32x4_kernel(f32x4 *__restrict__ dst,
                                                         const f32x4 *__restrict__ src, size_t n4)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride)
        __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

__global__ void synth_ids_kernel(int *out, size_t n, uint64_t seed, int V)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = (int)(mix64(seed + i) % (uint64_t)V);
}

// expf restatement exposed for the exhaustive check against glibc
__global__ void expf_check_kernel(uint32_t first_hi, int nhi, uint64_t *out)
{
    // one block per 65536-input chunk; out[chunk] = order-sensitive hash of results
    const uint32_t hi = first_hi + blockIdx.x;
    uint64_t h = 0;
    for (uint32_t lo = threadIdx.x; lo < 65536u; lo += blockDim.x) {
        const uint32_t ux = (hi << 16) | lo;
        const float r = glibc_expf(__uint_as_float(ux), kExp2Tab);
        uint32_t rb = __float_as_uint(r);
        if (r != r) rb = 0x7fc00000u;
        h += mix64(((uint64_t)ux << 32) | rb);
    }
    __shared__ uint64_t red[256];
    red[threadIdx.x] = h;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[blockIdx.x] = red[0];
    (void)nhi;
}

// Pre-pass of a call with a bias: the nonzero map and the maximum the
// sampler's stream filter bounds bias[e] with.  Bit e of bits is set unless
// bias[e] is +0.0 (x + +0.0 is what the filter computes for a clear bit, so
// its value is exact there; -0.0 is flagged, since x + -0.0 differs from
// x + +0.0 at x = -0.0).  part[block] is the largest order key over the
// block's flagged entries, all ones when one of them is a nan or -inf (their
// sums can be nans the bound would miss; the bound is then a nan and the
// rows take the nan path), 0 when none is flagged.  Blocks cover per_blk
// elements each (a multiple of 1024); each thread 4 consecutive elements per
// step, the 8 lanes of a word merged by shuffles.
__global__ __launch_bounds__(WG) void bias_prep_kernel(const float *bias, int V, int per_blk, uint32_t *bits,
                                                       uint32_t *part)
{
    __shared__ uint32_t red[NWAVE];
    const int lane = lane_id();
    const int beg = blockIdx.x * per_blk;
    const int end = min(V, beg + per_blk);
    uint32_t kmax = 0u;
    for (int base = beg; base < end; base += 4 * WG) {
        const int e0 = base + 4 * (int)threadIdx.x;
        uint32_t nib = 0u;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            if (e0 + c < end) {
                const float v = bias[e0 + c];
                if (__float_as_uint(v) != 0u) {
                    nib |= 1u << c;
                    kmax = max(kmax, (v != v || v == -INFINITY) ? 0xFFFFFFFFu : fkey(v));
                }
            }
        }
        uint32_t word = nib << (4 * (lane & 7));
        word |= (uint32_t)__shfl_xor((int)word, 1, 64);
        word |= (uint32_t)__shfl_xor((int)word, 2, 64);
        word |= (uint32_t)__shfl_xor((int)word, 4, 64);
        if ((lane & 7) == 0 && e0 < V) bits[e0 >> 5] = word;
    }
    kmax = wave_max_u(kmax);
    if (lane == 0) red[wave_id()] = kmax;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t m = red[0];
#pragma unroll
        for (int w = 1; w < NWAVE; ++w) m = max(m, red[w]);
        part[blockIdx.x] = m;
    }
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
struct lal_gpu_ctx {
    int device;
    int max_batch;
    int max_vocab;
    int ncu;  // compute units
    int forced_slices;  // LAL_GPU_SLICES at creation (0: choose per call)
    // LM head tuning overrides read at creation (0 / -1: the measured defaults)
    int lmh_wg;         // LAL_GPU_LMH_WG: workgroups per CU
    int lmh_xres;       // LAL_GPU_LMH_XRES: 0 disables the resident-activation kernel
    int lmh_pd;         // LAL_GPU_LMH_PD: W steps in flight (2 or 3)
    int list_ks;        // LAL_GPU_LIST_KS: rank of lal_gpu_lm_head_sample's bound (0: from k)
    int list_rows;      // LAL_GPU_LIST_ROWS: largest batch that uses the head's candidate lists
    int lmh_ksplit;     // LAL_GPU_LMH_KSPLIT: 0 disables the k-split head for 33..64 rows
    int head_qx;        // LAL_GPU_HEAD_QX: 1 lets the candidate head quantize up to 4 rows itself
    // slice lists (see KArgs): max_batch x FLAT_MAX entries, metadata for up
    // to MAX_SLICES slices per row, one arrival counter per row (zeroed here,
    // reset by every row's finisher)
    float *lst_val;
    int *lst_idx;
    int4 *lst_meta;
    unsigned *arrive;
    int *rr_ids;  // [max_batch][RERANK_MAX] ids kept by lal_gpu_lm_head_rerank's selection
    uint32_t *bias_bits;  // [ceil(max_vocab / 32)] nonzero map of a call's bias
    uint32_t *bias_part;  // [WG] its per-block maximum keys
    // lal_gpu_lm_head_sample's candidate state (zeroed here, cleared again by
    // the sampler after each use): per row (count, -, -, flags) every
    // HMETA_STRIDE int4 and 64 sample slots; the lists are lst_val / lst_idx
    int4 *hmeta;
    unsigned *hslots;
};

static thread_local hipError_t g_last_hip = hipSuccess;

static int hip_fail(hipError_t e)
{
    g_last_hip = e;
    return LAL_GPU_E_HIP;
}

#define LAL_HIP(call)                                  \
    do {                                               \
        hipError_t e_ = (call);                        \
        if (e_ != hipSuccess) return hip_fail(e_);     \
    } while (0)

extern "C" {

int lal_gpu_abi_version(void) { return LAL_GPU_ABI_VERSION; }

int lal_gpu_last_hip_error(void) { return (int)g_last_hip; }

const char *lal_gpu_strerror(int code)
{
    switch (code) {
    case LAL_GPU_OK: return "ok";
    case LAL_GPU_E_INVAL: return "invalid argument";
    case LAL_GPU_E_RANGE: return "size above a context or library limit";
    case LAL_GPU_E_HIP: return hipGetErrorString(g_last_hip);
    case LAL_GPU_E_NOMEM: return "out of device memory";
    case LAL_GPU_E_NODEV: return "no such device";
    default: return "unknown error";
    }
}

int lal_gpu_device_count(int *count)
{
    if (!count) return LAL_GPU_E_INVAL;
    LAL_HIP(hipGetDeviceCount(count));
    return LAL_GPU_OK;
}

int lal_gpu_set_device(int device)
{
    LAL_HIP(hipSetDevice(device));
    return LAL_GPU_OK;
}

int lal_gpu_create(lal_gpu_ctx **out, int device, int max_batch, int max_vocab)
{
    if (!out || max_batch <= 0 || max_vocab <= 0) return LAL_GPU_E_INVAL;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return LAL_GPU_E_NODEV;
    LAL_HIP(hipSetDevice(device));
    lal_gpu_ctx *c = (lal_gpu_ctx *)calloc(1, sizeof(lal_gpu_ctx));
    if (!c) return LAL_GPU_E_NOMEM;
    c->device = device;
    c->max_batch = max_batch;
    c->max_vocab = max_vocab;
    {
        int ncu = 0;
        if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || ncu <= 0)
            ncu = 256;
        c->ncu = ncu;
    }
    if (const char *env = getenv("LAL_GPU_SLICES")) c->forced_slices = std::max(0, atoi(env));
    c->lmh_xres = -1;
    if (const char *env = getenv("LAL_GPU_LMH_WG")) c->lmh_wg = std::max(0, atoi(env));
    if (const char *env = getenv("LAL_GPU_LMH_XRES")) c->lmh_xres = atoi(env) != 0;
    if (const char *env = getenv("LAL_GPU_LMH_PD")) c->lmh_pd = (atoi(env) == 3) ? 3 : 2;
    if (const char *env = getenv("LAL_GPU_LIST_KS")) c->list_ks = std::min(64, std::max(0, atoi(env)));
    // measured at [152064, 3584]: the lists win at 1 row (106 vs 112 us per
    // step) and at 16 rows (122 vs 127 us)
    c->list_rows = 16;
    // the k-split head's dynamic LDS goes past 64 KB
    c->lmh_ksplit = hipFuncSetAttribute((const void *)lm_head_ksplit_kernel<3>,
                                        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess &&
                    hipFuncSetAttribute((const void *)lm_head_ksplit_kernel<4>,
                                        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
    (void)hipGetLastError();
    if (const char *env = getenv("LAL_GPU_LMH_KSPLIT")) c->lmh_ksplit = c->lmh_ksplit && atoi(env) != 0;
    if (const char *env = getenv("LAL_GPU_LIST_ROWS")) c->list_rows = std::min(16, std::max(0, atoi(env)));
    // measured at [152064, 3584], B = 1: the separate one-round-trip
    // quantizer before the head is 2.4 us faster than the head's own
    if (const char *env = getenv("LAL_GPU_HEAD_QX")) c->head_qx = atoi(env) != 0;
    const size_t nl = (size_t)max_batch * FLAT_MAX;
    hipError_t e = hipMalloc((void **)&c->lst_val, nl * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&c->lst_idx, nl * sizeof(int));
    if (e == hipSuccess) e = hipMalloc((void **)&c->lst_meta, (size_t)max_batch * MAX_SLICES * sizeof(int4));
    if (e == hipSuccess) e = hipMalloc((void **)&c->arrive, (size_t)max_batch * sizeof(unsigned));
    if (e == hipSuccess) e = hipMemset(c->arrive, 0, (size_t)max_batch * sizeof(unsigned));
    if (e == hipSuccess) e = hipMalloc((void **)&c->rr_ids, (size_t)max_batch * RERANK_MAX * sizeof(int));
    if (e == hipSuccess) e = hipMalloc((void **)&c->bias_bits, (size_t)((max_vocab + 31) / 32) * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc((void **)&c->bias_part, (size_t)WG * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc((void **)&c->hmeta, (size_t)max_batch * HMETA_STRIDE * sizeof(int4));
    if (e == hipSuccess) e = hipMemset(c->hmeta, 0, (size_t)max_batch * HMETA_STRIDE * sizeof(int4));
    if (e == hipSuccess) e = hipMalloc((void **)&c->hslots, (size_t)max_batch * 64 * sizeof(unsigned));
    if (e == hipSuccess) e = hipMemset(c->hslots, 0, (size_t)max_batch * 64 * sizeof(unsigned));
    if (e != hipSuccess) {
        lal_gpu_destroy(c);
        return e == hipErrorOutOfMemory ? LAL_GPU_E_NOMEM : hip_fail(e);
    }
    *out = c;
    return LAL_GPU_OK;
}

void lal_gpu_destroy(lal_gpu_ctx *ctx)
{
    if (!ctx) return;
    int cur = -1;
    if (hipGetDevice(&cur) == hipSuccess && cur != ctx->device) (void)hipSetDevice(ctx->device);
    if (ctx->lst_val) (void)hipFree(ctx->lst_val);
    if (ctx->lst_idx) (void)hipFree(ctx->lst_idx);
    if (ctx->lst_meta) (void)hipFree(ctx->lst_meta);
    if (ctx->arrive) (void)hipFree(ctx->arrive);
    if (ctx->rr_ids) (void)hipFree(ctx->rr_ids);
    if (ctx->bias_bits) (void)hipFree(ctx->bias_bits);
    if (ctx->bias_part) (void)hipFree(ctx->bias_part);
    if (ctx->hmeta) (void)hipFree(ctx->hmeta);
    if (ctx->hslots) (void)hipFree(ctx->hslots);
    if (cur >= 0 && cur != ctx->device) (void)hipSetDevice(cur);
    free(ctx);
}

// Slices per row.  A slice costs a fixed setup and finish on top of its
// streaming, so rows are split only to give a small batch enough workgroups
// (about one per slot: 4 per CU): slices of at least 64 Ki elements, 32 Ki
// for at most 128 rows, 16 Ki for at most 16 rows; list capacity above k.
constexpr int TARGET_WGS = 1024;
// target: the workgroups resident at once (four per CU for the k <= 128
// instantiation, two for the large-k one, whose 66 KB of LDS leaves room for
// two): more slices than fill it once only add rounds of slice merging (512
// rows at k = 512 with one workgroup per CU: 363.5 us with 2 slices per row,
// 275.7 us with 1)
static int choose_slices(int batch, int vocab, int k_eff, int flat, int forced, int target)
{
    if (forced >= 1) return std::min(std::min(forced, MAX_SLICES), std::max(1, flat / (k_eff + 1)));
    // shortest slice per batch size (measured at 64 x 152064: 6 slices of
    // 25 K values 1.6 us faster than 4 of 38 K)
    const int min_len = (batch <= 16) ? 16384 : (batch <= 128) ? 24576 : 65536;
    int n = (target + batch - 1) / batch;
    n = std::min(n, std::max(1, vocab / min_len));
    n = std::min(n, std::max(1, flat / (k_eff + 1)));
    return std::max(1, std::min(n, MAX_SLICES));
}

}  // extern "C"

// Where a launch's slice lists live (a context's buffers or the static
// scratch of lal_gpu_sample_noalloc) and the device facts the launch needs.
struct ListTarget {
    int ncu;
    int forced_slices;
    int slice_rows;  // batches up to this many rows may be sliced; larger ones
                     // run one workgroup per row and touch no list
    float *lst_val;
    int *lst_idx;
    int4 *lst_meta;
    unsigned *arrive;
    uint32_t *bias_bits;  // nonzero map of the bias for up to bias_vocab ids
    uint32_t *bias_part;  // [WG]
    int bias_vocab;
    // list mode (an LM head's candidate lists in lst_val / lst_idx)
    bool list = false;
    int4 *hmeta = nullptr;
    unsigned *hslots = nullptr;
    int hks = 0;
};

static int launch_sample(const ListTarget &t, int batch, int vocab, const lal_gpu_sample_params *p,
                         const lal_gpu_sample_io *io, void *stream)
{
    if (!p || !io) return LAL_GPU_E_INVAL;
    if (batch <= 0 || vocab <= 0) return LAL_GPU_E_INVAL;
    if (!io->logits || !io->out_token || io->ld < vocab) return LAL_GPU_E_INVAL;
    const bool greedy = !(p->temperature > 0.0f) || p->top_k <= 0;
    // top_k is clamped to the vocabulary first, as the kernel and the
    // reference (qwen7b_server.c:236) do
    if (!greedy && std::min(p->top_k, vocab) > LAL_GPU_MAX_K) return LAL_GPU_E_RANGE;
    if (!greedy && !io->uniforms) return LAL_GPU_E_INVAL;
    if (io->history && (io->history_ld <= 0 || io->history_ld > LAL_GPU_MAX_HISTORY))
        return io->history_ld > LAL_GPU_MAX_HISTORY ? LAL_GPU_E_RANGE : LAL_GPU_E_INVAL;
    if (io->allow_bits && io->allow_ld < (vocab + 31) / 32) return LAL_GPU_E_INVAL;
    if (p->n_ban_ids < 0 || p->n_ban_ids > LAL_GPU_MAX_BAN_IDS) return LAL_GPU_E_RANGE;
    if (p->n_ban_ids > 0 && !p->ban_ids) return LAL_GPU_E_INVAL;
    if (p->variant != LAL_GPU_VARIANT_BASIC && p->variant != LAL_GPU_VARIANT_FILTERED)
        return LAL_GPU_E_INVAL;
    if (io->cand_ld < 0 ||
        (io->cand_ld > 0 && !io->cand_ids && !io->cand_probs && !io->cand_kept && !io->cand_vals))
        return LAL_GPU_E_INVAL;
    if (io->out_history_vals && !io->history) return LAL_GPU_E_INVAL;

    KArgs A;
    memset(&A, 0, sizeof A);
    A.logits = io->logits;
    A.logits_w = io->logits;
    A.ld = io->ld;
    A.V = vocab;
    A.hist = io->history;
    A.hist_ld = io->history ? io->history_ld : 0;
    A.hist_len = io->history ? io->history_len : nullptr;
    A.allow = io->allow_bits;
    A.allow_ld = io->allow_ld;
    A.bias = io->bias;
    A.uniforms = io->uniforms;
    A.out_token = io->out_token;
    A.out_thr = io->out_threshold;
    A.out_ncand = io->out_n_cand;
    A.out_nkept = io->out_n_kept;
    A.out_sum = io->out_sum;
    A.cand_ld = io->cand_ld;
    A.cand_ids = io->cand_ids;
    A.cand_probs = io->cand_probs;
    A.cand_kept = io->cand_kept;
    A.cand_vals = io->cand_vals;
    A.out_hvals = io->out_history_vals;
    A.ban_ids = p->ban_ids;
    A.n_ban = p->n_ban_ids;
    A.last_tokens = io->last_tokens;
    A.T = p->temperature;
    A.top_p = p->top_p;
    A.pen = p->rep_penalty;
    A.k = p->top_k;
    A.variant = p->variant;
    A.flags = p->flags;
    A.ban_last = p->ban_last;
    A.ban_repeat = p->ban_repeat;
    A.mask_recent = p->mask_recent;
    A.greedy = greedy ? 1 : 0;
    A.fallback = (p->flags & LAL_GPU_F_FALLBACK_ZERO) ? 0 : vocab - 1;
    const bool has_hist = io->history != nullptr;
    A.apply_pen = (p->rep_penalty > 1.0f && has_hist &&
                   (p->variant == LAL_GPU_VARIANT_FILTERED || !greedy)) ? 1 : 0;
    // bans act on the pool; on greedy rows only with F_GREEDY_FILTER
    const bool bans_apply = !greedy || (p->flags & LAL_GPU_F_GREEDY_FILTER);
    const bool has_last = has_hist || io->last_tokens;
    A.any_bans = (bans_apply && ((has_last && p->ban_last) || (has_hist && p->ban_repeat > 0) ||
                                 p->n_ban_ids > 0)) ? 1 : 0;
    if (!has_hist) {
        A.ban_repeat = 0;
        A.mask_recent = 0;
    }
    if (!has_last) A.ban_last = 0;
    if (!A.any_bans) {
        A.ban_last = 0;
        A.ban_repeat = 0;
        A.n_ban = 0;
        A.last_tokens = nullptr;
    }

    hipStream_t s = (hipStream_t)stream;
    const int k_eff = greedy ? 1 : std::min(p->top_k, vocab);
    const bool small = k_eff <= K_SMALL_MAX;
    const int flat = NWAVE * (small ? CAPW_SMALL : CAPW_LARGE);
    A.batch = batch;
    A.nslice = (batch <= t.slice_rows)
                   ? choose_slices(batch, vocab, k_eff, flat, t.forced_slices, small ? TARGET_WGS : TARGET_WGS / 2)
                   : 1;
    if (t.list) {
        if (A.bias || A.allow) return LAL_GPU_E_INVAL;
        A.nslice = 1;
        A.hmeta = t.hmeta;
        A.hslots = t.hslots;
        A.hcap = FLAT_MAX;
        A.hks = t.hks;
    }
    A.ncu = t.ncu;
    A.lcap = flat / A.nslice;
    // a slice list must hold more than k values (see the finisher): always
    // true by choose_slices, checked so that the kernel's overflow branch
    // stays unreachable
    if (A.nslice > 1 && A.lcap <= k_eff) return LAL_GPU_E_RANGE;
    // sliced batches that fill the GPU (measured: 512 x 152064 with 2 slices
    // per row, 86.9 -> 83.9 us; one workgroup per row is faster with the
    // fixed step)
    A.prio_rotate = (A.nslice > 1 && batch >= 64) ? 1 : 0;
    A.lst_val = t.lst_val;
    A.lst_idx = t.lst_idx;
    A.lst_meta = t.lst_meta;
    A.arrive = t.arrive;
    if (A.bias) {
        // the bias's nonzero map and maxima, ahead of the sampler in the stream
        if (vocab > t.bias_vocab) return LAL_GPU_E_RANGE;
        const int per_blk = std::max(4 * WG, (int)((((long long)vocab + WG - 1) / WG + 4 * WG - 1) /
                                                  (4 * WG) * (4 * WG)));
        A.bias_nparts = (vocab + per_blk - 1) / per_blk;
        A.bias_bits = t.bias_bits;
        A.bias_part = t.bias_part;
        hipLaunchKernelGGL(bias_prep_kernel, dim3((unsigned)A.bias_nparts), dim3(WG), 0, s, A.bias, vocab, per_blk,
                           t.bias_bits, t.bias_part);
    }
    const dim3 grid((unsigned)(((batch + 7) / 8) * 8 * A.nslice)), block(WG);
#define LAL_LAUNCH(HB, HA)                                                                   \
    do {                                                                                     \
        if (small)                                                                           \
            hipLaunchKernelGGL((sample_rows_kernel<HB, HA, CAPW_SMALL>), grid, block, 0, s, A); \
        else                                                                                 \
            hipLaunchKernelGGL((sample_rows_kernel<HB, HA, CAPW_LARGE>), grid, block, 0, s, A); \
    } while (0)
    if (t.list) {
        if (small)
            hipLaunchKernelGGL((sample_rows_kernel<false, false, CAPW_SMALL, true>), grid, block, 0, s, A);
        else
            hipLaunchKernelGGL((sample_rows_kernel<false, false, CAPW_LARGE, true>), grid, block, 0, s, A);
    } else if (A.bias && A.allow) LAL_LAUNCH(true, true);
    else if (A.bias) LAL_LAUNCH(true, false);
    else if (A.allow) LAL_LAUNCH(false, true);
    else LAL_LAUNCH(false, false);
#undef LAL_LAUNCH
    LAL_HIP(hipGetLastError());
    return LAL_GPU_OK;
}

// ---- the sampler without allocation ---------------------------------------
// Candidate lists and arrival counters of up to LAL_GPU_NOALLOC_MAX_ROWS sliced
// rows, in one file-scope device array: each GPU the library runs on holds its
// own copy (about 3.3 MB) until the process ends.  Host code never uses the
// array's name as an address: its device address comes from
// hipGetSymbolAddress, once per device, with that device current.
struct NoallocScratch {
    float lst_val[LAL_GPU_NOALLOC_MAX_ROWS * FLAT_MAX];
    int lst_idx[LAL_GPU_NOALLOC_MAX_ROWS * FLAT_MAX];
    int4 lst_meta[LAL_GPU_NOALLOC_MAX_ROWS * MAX_SLICES];
    unsigned arrive[LAL_GPU_NOALLOC_MAX_ROWS];
    uint32_t bias_bits[LAL_GPU_NOALLOC_MAX_BIAS_VOCAB / 32];
    uint32_t bias_part[WG];
};
static __device__ __align__(256) NoallocScratch scratch;

namespace {
// the arrival counters start at zero (each row's finisher resets its own)
__global__ void clear_u32_kernel(unsigned *p, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

constexpr int NOALLOC_MAX_DEVICES = 64;
struct NoallocDevice {
    std::once_flag once;
    int rc = LAL_GPU_OK;
    int ncu = 0;
    int forced_slices = 0;
    NoallocScratch *ptr = nullptr;  // this device's copy of `scratch`
};
NoallocDevice g_noalloc[NOALLOC_MAX_DEVICES];
}  // namespace

extern "C" {

int lal_gpu_sample_noalloc(int batch, int vocab, const lal_gpu_sample_params *params,
                           const lal_gpu_sample_io *io, void *stream)
{
    int dev = -1;
    LAL_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return LAL_GPU_E_NODEV;
    NoallocDevice &d = g_noalloc[dev];
    std::call_once(d.once, [&]() {
        NoallocScratch *ptr = nullptr;
        hipError_t e = hipGetSymbolAddress((void **)&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            d.rc = hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol);
            return;
        }
        int ncu = 0;
        if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0)
            ncu = 256;
        d.ncu = ncu;
        if (const char *env = getenv("LAL_GPU_SLICES")) d.forced_slices = std::max(0, atoi(env));
        hipLaunchKernelGGL(clear_u32_kernel, dim3((LAL_GPU_NOALLOC_MAX_ROWS + 255) / 256), dim3(256), 0,
                           (hipStream_t)stream, ptr->arrive, LAL_GPU_NOALLOC_MAX_ROWS);
        e = hipGetLastError();
        if (e != hipSuccess) {
            d.rc = hip_fail(e);
            return;
        }
        d.ptr = ptr;
    });
    if (d.rc != LAL_GPU_OK || !d.ptr) return d.rc != LAL_GPU_OK ? d.rc : LAL_GPU_E_HIP;
    if (batch > LAL_GPU_NOALLOC_MAX_ROWS && d.forced_slices > 1) return LAL_GPU_E_RANGE;
    ListTarget t;
    t.ncu = d.ncu;
    t.forced_slices = d.forced_slices;
    t.slice_rows = LAL_GPU_NOALLOC_MAX_ROWS;
    t.lst_val = d.ptr->lst_val;
    t.lst_idx = d.ptr->lst_idx;
    t.lst_meta = d.ptr->lst_meta;
    t.arrive = d.ptr->arrive;
    t.bias_bits = d.ptr->bias_bits;
    t.bias_part = d.ptr->bias_part;
    t.bias_vocab = LAL_GPU_NOALLOC_MAX_BIAS_VOCAB;
    return launch_sample(t, batch, vocab, params, io, stream);
}

int lal_gpu_sample(lal_gpu_ctx *ctx, int batch, int vocab, const lal_gpu_sample_params *p,
                   const lal_gpu_sample_io *io, void *stream)
{
    if (!ctx) return LAL_GPU_E_INVAL;
    if (batch > ctx->max_batch || vocab > ctx->max_vocab) return LAL_GPU_E_RANGE;
    ListTarget t;
    t.ncu = ctx->ncu;
    t.forced_slices = ctx->forced_slices;
    t.slice_rows = ctx->max_batch;
    t.lst_val = ctx->lst_val;
    t.lst_idx = ctx->lst_idx;
    t.lst_meta = ctx->lst_meta;
    t.arrive = ctx->arrive;
    t.bias_bits = ctx->bias_bits;
    t.bias_part = ctx->bias_part;
    t.bias_vocab = ctx->max_vocab;
    return launch_sample(t, batch, vocab, p, io, stream);
}

int lal_gpu_sample_finish(lal_gpu_ctx *ctx, int batch, int vocab, const lal_gpu_sample_params *p,
                          const lal_gpu_finish_io *io, void *stream)
{
    if (!ctx || !p || !io || batch <= 0 || vocab <= 0) return LAL_GPU_E_INVAL;
    if (batch > ctx->max_batch) return LAL_GPU_E_RANGE;
    if (!io->n_cand || !io->cand_ids || !io->cand_vals || !io->keep || !io->out_token || io->cand_ld <= 0)
        return LAL_GPU_E_INVAL;
    if (p->variant != LAL_GPU_VARIANT_BASIC && p->variant != LAL_GPU_VARIANT_FILTERED) return LAL_GPU_E_INVAL;
    if (!(p->temperature > 0.0f)) return LAL_GPU_E_INVAL;  // greedy rows have no softmax to finish
    FinishArgs F;
    F.V = vocab;
    F.variant = p->variant;
    F.flags = p->flags;
    F.T = p->temperature;
    F.cand_ld = io->cand_ld;
    F.n_cand = io->n_cand;
    F.ids = io->cand_ids;
    F.vals = io->cand_vals;
    F.keep = io->keep;
    F.uniforms = io->uniforms;
    F.out_token = io->out_token;
    F.out_n_kept = io->out_n_kept;
    F.out_sum = io->out_sum;
    hipLaunchKernelGGL(finish_rows_kernel, dim3(batch), dim3(WG), 0, (hipStream_t)stream, F);
    LAL_HIP(hipGetLastError());
    return LAL_GPU_OK;
}

int lal_gpu_quantize_x(lal_gpu_ctx *ctx, const float *d_x, int batch, int n, int mode, int8_t *d_xq,
                       float *d_sx, void *stream)
{
    if (!ctx || !d_x || !d_xq || !d_sx || batch <= 0 || n <= 0 || (mode != 0 && mode != 1))
        return LAL_GPU_E_INVAL;
    if (n <= QXF_MAXN)
        hipLaunchKernelGGL(quantize_x_fast_kernel, dim3(batch), dim3(256), 0, (hipStream_t)stream, d_x, n, mode,
                           d_xq, d_sx);
    else
        hipLaunchKernelGGL(quantize_x_kernel, dim3(batch), dim3(256), 0, (hipStream_t)stream, d_x, n, mode,
                           d_xq, d_sx);
    LAL_HIP(hipGetLastError());
    return LAL_GPU_OK;
}

int lal_gpu_lm_head_q8(lal_gpu_ctx *ctx, const int8_t *d_xq, const float *d_sx, int batch, int n,
                       const int8_t *d_w, const float *d_sw, int vocab, float *d_logits, int ld,
                       void *stream)
{
    if (!ctx || !d_xq || !d_sx || !d_w || !d_sw || !d_logits) return LAL_GPU_E_INVAL;
    if (batch <= 0 || n <= 0 || vocab <= 0 || ld < vocab) return LAL_GPU_E_INVAL;
    hipStream_t s = (hipStream_t)stream;
    if (((uintptr_t)d_xq & 15) || ((uintptr_t)d_w & 15) || (n & 15)) {
        // rows not 16-byte aligned: byte-load kernel
        hipLaunchKernelGGL(lm_head_scalar_kernel, dim3((vocab + 3) / 4), dim3(256), 0, s, d_xq, d_sx,
                           n, d_w, d_sw, vocab, d_logits, ld, batch);
        LAL_HIP(hipGetLastError());
        return LAL_GPU_OK;
    }
    if (batch > LMH_MAXB) {
        int per_cu = 4;
        if (ctx->lmh_wg > 0) per_cu = ctx->lmh_wg;
        const unsigned nwg = (unsigned)std::min(per_cu * ctx->ncu, (vocab + LMM_TILE_V - 1) / LMM_TILE_V);
        for (int b0 = 0; b0 < batch; b0 += LMM_MAXB) {
            const int nb = std::min(LMM_MAXB, batch - b0);
            const dim3 g2(nwg), blk(64 * LMM_WAVES);
            switch ((nb + 15) / 16) {
            case 1: hipLaunchKernelGGL(lm_head_mfma_kernel<1>, g2, blk, 0, s, d_xq, d_sx, n, d_w, d_sw, vocab, d_logits, ld, b0, nb); break;
            case 2: hipLaunchKernelGGL(lm_head_mfma_kernel<2>, g2, blk, 0, s, d_xq, d_sx, n, d_w, d_sw, vocab, d_logits, ld, b0, nb); break;
            case 3: hipLaunchKernelGGL(lm_head_mfma_kernel<3>, g2, blk, 0, s, d_xq, d_sx, n, d_w, d_sw, vocab, d_logits, ld, b0, nb); break;
            default: hipLaunchKernelGGL(lm_head_mfma_kernel<4>, g2, blk, 0, s, d_xq, d_sx, n, d_w, d_sw, vocab, d_logits, ld, b0, nb); break;
            }
            LAL_HIP(hipGetLastError());
        }
        return LAL_GPU_OK;
    }
    const int waves = (vocab + LMH_ROWS - 1) / LMH_ROWS;
    const dim3 grid((waves + 3) / 4), block(256);
    for (int b0 = 0; b0 < batch; b0 += LMH_MAXB) {
        const int nb = std::min(LMH_MAXB, batch - b0);
        switch (nb) {
        case 1: hipLaunchKernelGGL(lm_head_dot4_kernel<1>, grid, block, 0, s, d_xq, d_sx, n, d_w, d_sw, vocab, d_logits, ld, b0); break;
        case 2: hipLaunchKernelGGL(lm_head_dot4_kernel<2>, grid, block, 0, s, d_xq, d_sx, n, d_w, d_sw, vocab, d_logits, ld, b0); break;
        case 3: hipLaunchKernelGGL(lm_head_dot4_kernel<3>, grid, block, 0, s, d_xq, d_sx, n, d_w, d_sw, vocab, d_logits, ld, b0); break;
        case 4: hipLaunchKernelGGL(lm_head_dot4_kernel<4>, grid, block, 0, s, d_xq, d_sx, n, d_w, d_sw, vocab, d_logits, ld, b0); break;
        case 5: hipLaunchKernelGGL(lm_head_dot4_kernel<5>, grid, block, 0, s, d_xq, d_sx, n, d_w, d_sw, vocab, d_logits, ld, b0); break;
        case 6: hipLaunchKernelGGL(lm_head_dot4_kernel<6>, grid, block, 0, s, d_xq, d_sx, n, d_w, d_sw, vocab, d_logits, ld, b0); break;
        case 7: hipLaunchKernelGGL(lm_head_dot4_kernel<7>, grid, block, 0, s, d_xq, d_sx, n, d_w, d_sw, vocab, d_logits, ld, b0); break;
        default: hipLaunchKernelGGL(lm_head_dot4_kernel<8>, grid, block, 0, s, d_xq, d_sx, n, d_w, d_sw, vocab, d_logits, ld, b0); break;
        }
        LAL_HIP(hipGetLastError());
    }
    return LAL_GPU_OK;
}

size_t lal_gpu_q8_packed_bytes(int vocab, int n)
{
    if (vocab <= 0 || n <= 0) return 0;
    return (size_t)((vocab + 15) / 16) * (size_t)((n + 63) / 64) * 1024u;
}

int lal_gpu_pack_q8(lal_gpu_ctx *ctx, const int8_t *d_w, int vocab, int n, int8_t *d_wpk, void *stream)
{
    if (!ctx || !d_w || !d_wpk || vocab <= 0 || n <= 0) return LAL_GPU_E_INVAL;
    if ((uintptr_t)d_wpk & 15) return LAL_GPU_E_INVAL;
    const size_t units = lal_gpu_q8_packed_bytes(vocab, n) / 16;
    const size_t nblk = (units + 255) / 256;
    if (nblk > 0x7fffffffu) return LAL_GPU_E_RANGE;
    hipLaunchKernelGGL(pack_q8_kernel, dim3((unsigned)nblk), dim3(256), 0, (hipStream_t)stream, d_w, vocab, n,
                       d_wpk);
    LAL_HIP(hipGetLastError());
    return LAL_GPU_OK;
}

int lal_gpu_quantize_w_q8(lal_gpu_ctx *ctx, const float *d_w, int vocab, int n, int8_t *d_wq, int8_t *d_wpk,
                          float *d_sw, void *stream)
{
    if (!ctx || !d_w || !d_sw || vocab <= 0 || n <= 0 || (!d_wq && !d_wpk)) return LAL_GPU_E_INVAL;
    if (d_wpk && ((uintptr_t)d_wpk & 15)) return LAL_GPU_E_INVAL;
    hipStream_t s = (hipStream_t)stream;
    int8_t *q = d_wq;
    if (!q) LAL_HIP(hipMallocAsync((void **)&q, (size_t)vocab * n, s));
    hipLaunchKernelGGL(quantize_w_kernel, dim3(vocab), dim3(256), 0, s, d_w, n, q, d_sw);
    hipError_t e = hipGetLastError();
    int rc = (e == hipSuccess) ? LAL_GPU_OK : hip_fail(e);
    if (rc == LAL_GPU_OK && d_wpk) rc = lal_gpu_pack_q8(ctx, q, vocab, n, d_wpk, stream);
    if (!d_wq) {
        const hipError_t f = hipFreeAsync(q, s);
        if (rc == LAL_GPU_OK && f != hipSuccess) rc = hip_fail(f);
    }
    return rc;
}

int lal_gpu_lm_head_q8_packed(lal_gpu_ctx *ctx, const int8_t *d_xq, const float *d_sx, int batch, int n,
                              const int8_t *d_wpk, const float *d_sw, int vocab, float *d_logits, int ld,
                              void *stream)
{
    if (!ctx || !d_xq || !d_sx || !d_wpk || !d_sw || !d_logits) return LAL_GPU_E_INVAL;
    if (batch <= 0 || n <= 0 || vocab <= 0 || ld < vocab) return LAL_GPU_E_INVAL;
    if (((uintptr_t)d_xq & 15) || ((uintptr_t)d_wpk & 15) || (n & 15)) return LAL_GPU_E_INVAL;
    hipStream_t s = (hipStream_t)stream;
    const int ntile = (vocab + 15) / 16;
    for (int b0 = 0; b0 < batch; b0 += LMM_MAXB) {
        const int nb = std::min(LMM_MAXB, batch - b0);
        const int mt = (nb + 15) / 16;
        // up to 16 rows: the activations resident in LDS (64 KB: 2 workgroups per CU)
        bool xres = mt == 1 && n <= LMX_MAXN;
        if (ctx->lmh_xres == 0) xres = false;
        int per_cu = xres ? 2 : (mt <= 2) ? 4 : 2;  // workgroups per CU (measured best at each shape)
        if (ctx->lmh_wg > 0) per_cu = ctx->lmh_wg;
        const unsigned nwg = (unsigned)std::max(1, std::min(per_cu * ctx->ncu, (ntile + LMM_WAVES - 1) / LMM_WAVES));
        const dim3 g2(nwg), blk(64 * LMM_WAVES);
        if (xres) {
            hipLaunchKernelGGL(lm_head_packed_xres_kernel<false>, g2, blk, 0, s, d_xq, d_sx, n, d_wpk, d_sw, vocab,
                               d_logits, ld, b0, nb, HeadCand{}, HeadQuant{});
            LAL_HIP(hipGetLastError());
            continue;
        }
        // 33..64 rows: k split in two halves with the activations resident
        // (one workgroup of 8 waves per CU); each half at least four passes
        // of 256 k-bytes, every workgroup's share of tiles within LMK_MAXT
        // per wave, the LDS within the CU's 160 KB
        const int kwg = ctx->ncu;
        const int npass = (n + LMM_KC - 1) / LMM_KC, P0 = (npass + 1) / 2;
        const size_t klds = lmk_lds_bytes(mt, P0);
        const bool ksplit = ctx->lmh_ksplit && mt >= 3 && npass - P0 >= 4 && klds <= 160 * 1024 &&
                            mt * 16 * 16 * P0 <= LMK_XPT * 64 * LMK_WAVES &&
                            (ntile + kwg - 1) / kwg <= LMK_MAXT * LMK_WAVES;
        if (ksplit) {
            if (mt == 3)
                hipLaunchKernelGGL(lm_head_ksplit_kernel<3>, dim3(kwg), dim3(64 * LMK_WAVES), klds, s, d_xq, d_sx,
                                   n, d_wpk, d_sw, vocab, d_logits, ld, b0, nb);
            else
                hipLaunchKernelGGL(lm_head_ksplit_kernel<4>, dim3(kwg), dim3(64 * LMK_WAVES), klds, s, d_xq, d_sx,
                                   n, d_wpk, d_sw, vocab, d_logits, ld, b0, nb);
            LAL_HIP(hipGetLastError());
            continue;
        }
        int pd = (mt <= 2) ? 2 : 3;  // W steps in flight per wave
        if (ctx->lmh_pd) pd = ctx->lmh_pd;
#define LAL_LMH(M, D) \
    hipLaunchKernelGGL((lm_head_packed_kernel<M, D>), g2, blk, 0, s, d_xq, d_sx, n, d_wpk, d_sw, vocab, d_logits, ld, b0, nb)
        switch (mt * 4 + pd) {
        case 6: LAL_LMH(1, 2); break;
        case 7: LAL_LMH(1, 3); break;
        case 10: LAL_LMH(2, 2); break;
        case 11: LAL_LMH(2, 3); break;
        case 14: LAL_LMH(3, 2); break;
        case 15: LAL_LMH(3, 3); break;
        case 18: LAL_LMH(4, 2); break;
        default: LAL_LMH(4, 3); break;
        }
#undef LAL_LMH
        LAL_HIP(hipGetLastError());
    }
    return LAL_GPU_OK;
}

int lal_gpu_lm_head_sample(lal_gpu_ctx *ctx, const float *d_x, int batch, int n, int8_t *d_xq, float *d_sx,
                           const int8_t *d_wpk, const float *d_sw, int vocab, float *d_logits, int ld,
                           const lal_gpu_sample_params *p, const lal_gpu_sample_io *io, void *stream)
{
    if (!ctx || !d_x || !d_xq || !d_sx || !d_wpk || !d_sw || !d_logits || !p || !io) return LAL_GPU_E_INVAL;
    if (batch <= 0 || n <= 0 || vocab <= 0 || ld < vocab) return LAL_GPU_E_INVAL;
    if (batch > ctx->max_batch || vocab > ctx->max_vocab) return LAL_GPU_E_RANGE;
    if (((uintptr_t)d_xq & 15) || ((uintptr_t)d_wpk & 15) || (n & 15)) return LAL_GPU_E_INVAL;
    lal_gpu_sample_io sio = *io;
    sio.logits = d_logits;
    sio.ld = ld;
    int rc = LAL_GPU_OK;
    // candidate lists from the head: up to 16 rows (activations resident),
    // no bias or allow mask (the list holds raw logits), and a sample bound
    // (ks <= 64 slots) for the row's k
    const bool greedy = !(p->temperature > 0.0f) || p->top_k <= 0;
    const int k_eff = greedy ? 1 : std::min(std::max(p->top_k, 1), vocab);
    const int ntile = (vocab + 15) / 16;
    const unsigned nwg = (unsigned)std::max(1, std::min((ctx->lmh_wg > 0 ? ctx->lmh_wg : 2) * ctx->ncu,
                                                        (ntile + LMM_WAVES - 1) / LMM_WAVES));
    const double ns = std::min((double)vocab, 16.0 * std::min((double)ntile, (double)nwg * LMM_WAVES));
    const double lam = (double)k_eff * ns / (double)vocab;
    const int ks = ctx->list_ks > 0 ? ctx->list_ks : (int)std::ceil(lam + 6.0 * std::sqrt(lam) + 6.0);
    // (a tile spans at least four 256-byte passes of k: at most one finished
    // tile per group of four steps waits for the candidate code)
    const bool cand = batch <= ctx->list_rows && n <= LMX_MAXN && n > 3 * LMM_KC && ctx->lmh_xres != 0 &&
                      !io->allow_bits && !io->bias && ks <= 64 && k_eff <= LAL_GPU_MAX_K;
    // up to QX_ROWS rows the head quantizes the activations itself
    const bool qx_in = ctx->head_qx && cand && batch <= QX_ROWS && ((uintptr_t)d_x & 15) == 0;
    if (!qx_in) {
        rc = lal_gpu_quantize_x(ctx, d_x, batch, n, 0, d_xq, d_sx, stream);
        if (rc != LAL_GPU_OK) return rc;
    }
    if (!cand) {
        rc = lal_gpu_lm_head_q8_packed(ctx, d_xq, d_sx, batch, n, d_wpk, d_sw, vocab, d_logits, ld, stream);
        if (rc != LAL_GPU_OK) return rc;
        return lal_gpu_sample(ctx, batch, vocab, p, &sio, stream);
    }
    HeadCand C;
    C.hmeta = ctx->hmeta;
    C.hslots = ctx->hslots;
    C.lval = ctx->lst_val;
    C.lidx = ctx->lst_idx;
    C.hcap = FLAT_MAX;
    C.ks = ks;
    HeadQuant HQ;
    HQ.x = qx_in ? d_x : nullptr;
    HQ.xq = d_xq;
    HQ.sx = d_sx;
    hipLaunchKernelGGL(lm_head_packed_xres_kernel<true>, dim3(nwg), dim3(64 * LMM_WAVES), 0, (hipStream_t)stream,
                       d_xq, d_sx, n, d_wpk, d_sw, vocab, d_logits, ld, 0, batch, C, HQ);
    LAL_HIP(hipGetLastError());
    ListTarget t;
    t.ncu = ctx->ncu;
    t.forced_slices = 1;
    t.slice_rows = ctx->max_batch;
    t.lst_val = ctx->lst_val;
    t.lst_idx = ctx->lst_idx;
    t.lst_meta = ctx->lst_meta;
    t.arrive = ctx->arrive;
    t.bias_bits = ctx->bias_bits;
    t.bias_part = ctx->bias_part;
    t.bias_vocab = ctx->max_vocab;
    t.list = true;
    t.hmeta = ctx->hmeta;
    t.hslots = ctx->hslots;
    t.hks = ks;
    return launch_sample(t, batch, vocab, p, &sio, stream);
}

int lal_gpu_lm_head_rerank(lal_gpu_ctx *ctx, const float *d_x, int batch, int n, const int8_t *d_wq,
                           const float *d_ws, int vocab, int rerank_n, float *d_logits, int ld, void *stream)
{
    if (!ctx || !d_x || !d_wq || !d_ws || !d_logits) return LAL_GPU_E_INVAL;
    if (batch <= 0 || n <= 0 || vocab <= 0 || rerank_n <= 0 || ld < vocab) return LAL_GPU_E_INVAL;
    if (rerank_n > RERANK_MAX || n > RERANK_MAXN || vocab > RR_VPT * RR_WG) return LAL_GPU_E_RANGE;
    if (batch > ctx->max_batch) return LAL_GPU_E_RANGE;
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(rerank_select_kernel, dim3(batch), dim3(RR_WG), 0, s, vocab, rerank_n, d_logits, ld,
                       ctx->rr_ids);
    LAL_HIP(hipGetLastError());
    const int per = std::min(RR_PER, RR_STAGE / ((n + 4) & ~3));
    const int r_eff = std::min(rerank_n, vocab);
    hipLaunchKernelGGL(rerank_score_kernel, dim3(batch, (r_eff + per - 1) / per), dim3(RR_SCORE_WG), 0, s, d_x, n,
                       d_wq, d_ws, vocab, rerank_n, d_logits, ld, (const int *)ctx->rr_ids);
    LAL_HIP(hipGetLastError());
    return LAL_GPU_OK;
}

void lal_gpu_uniforms_rand(unsigned seed, int n, float *out, int gpt2)
{
    srand(seed);
    for (int i = 0; i < n; i++) {
        if (gpt2) out[i] = (float)(rand() % 1000000) / 1000000.0f;
        else out[i] = (float)rand() / (float)RAND_MAX;
    }
}

int lal_gpu_malloc(void **d_ptr, size_t bytes)
{
    if (!d_ptr) return LAL_GPU_E_INVAL;
    hipError_t e = hipMalloc(d_ptr, bytes ? bytes : 1);
    if (e == hipErrorOutOfMemory) {
        g_last_hip = e;
        return LAL_GPU_E_NOMEM;
    }
    LAL_HIP(e);
    return LAL_GPU_OK;
}

int lal_gpu_free(void *d_ptr)
{
    LAL_HIP(hipFree(d_ptr));
    return LAL_GPU_OK;
}

int lal_gpu_memcpy_h2d(void *d_dst, const void *h_src, size_t bytes, void *stream)
{
    LAL_HIP(hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream));
    return LAL_GPU_OK;
}

int lal_gpu_memcpy_d2h(void *h_dst, const void *d_src, size_t bytes, void *stream)
{
    LAL_HIP(hipMemcpyAsync(h_dst, d_src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream));
    LAL_HIP(hipStreamSynchronize((hipStream_t)stream));
    return LAL_GPU_OK;
}

int lal_gpu_memcpy_d2d(void *d_dst, const void *d_src, size_t bytes, void *stream)
{
    LAL_HIP(hipMemcpyAsync(d_dst, d_src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream));
    return LAL_GPU_OK;
}

int lal_gpu_memset(void *d_dst, int value, size_t bytes, void *stream)
{
    LAL_HIP(hipMemsetAsync(d_dst, value, bytes, (hipStream_t)stream));
    return LAL_GPU_OK;
}

int lal_gpu_stream_create(void **stream)
{
    if (!stream) return LAL_GPU_E_INVAL;
    hipStream_t s;
    LAL_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = (void *)s;
    return LAL_GPU_OK;
}

int lal_gpu_stream_destroy(void *stream)
{
    LAL_HIP(hipStreamDestroy((hipStream_t)stream));
    return LAL_GPU_OK;
}

int lal_gpu_stream_sync(void *stream)
{
    LAL_HIP(hipStreamSynchronize((hipStream_t)stream));
    return LAL_GPU_OK;
}

int lal_gpu_device_sync(void)
{
    LAL_HIP(hipDeviceSynchronize());
    return LAL_GPU_OK;
}

int lal_gpu_event_create(void **event)
{
    if (!event) return LAL_GPU_E_INVAL;
    hipEvent_t e;
    LAL_HIP(hipEventCreate(&e));
    *event = (void *)e;
    return LAL_GPU_OK;
}

int lal_gpu_event_destroy(void *event)
{
    LAL_HIP(hipEventDestroy((hipEvent_t)event));
    return LAL_GPU_OK;
}

int lal_gpu_event_record(void *event, void *stream)
{
    LAL_HIP(hipEventRecord((hipEvent_t)event, (hipStream_t)stream));
    return LAL_GPU_OK;
}

int lal_gpu_event_elapsed_ms(float *ms, void *start, void *stop)
{
    if (!ms) return LAL_GPU_E_INVAL;
    LAL_HIP(hipEventSynchronize((hipEvent_t)stop));
    LAL_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
    return LAL_GPU_OK;
}

// ---- synthetic workloads ---------------------------------------------------
static dim3 grid_for(size_t n)
{
    size_t blocks = (n + 255) / 256;
    if (blocks > 65535) blocks = 65535;
    if (blocks < 1) blocks = 1;
    return dim3((unsigned)blocks);
}

int lal_gpu_synth_gauss(float *d_out, int batch, int vocab, int ld, unsigned long long seed, float sigma,
                        float offset_range, int n_outliers, float outlier_value, void *stream)
{
    if (!d_out || batch <= 0 || vocab <= 0 || ld < vocab || n_outliers < 0 || n_outliers > 256)
        return LAL_GPU_E_INVAL;
    const dim3 grid((vocab + 256 * 16 - 1) / (256 * 16), batch);
    hipLaunchKernelGGL(synth_gauss_kernel, grid, dim3(256), 0, (hipStream_t)stream, d_out, vocab, ld,
                       (uint64_t)seed, sigma, offset_range, n_outliers, outlier_value);
    LAL_HIP(hipGetLastError());
    return LAL_GPU_OK;
}

int lal_gpu_synth_zipf(float *d_out, int batch, int vocab, int ld, unsigned long long seed, float slope,
                       float noise, void *stream)
{
    if (!d_out || batch <= 0 || vocab <= 0 || ld < vocab) return LAL_GPU_E_INVAL;
    const dim3 grid((vocab + 256 * 16 - 1) / (256 * 16), batch);
    hipLaunchKernelGGL(synth_zipf_kernel, grid, dim3(256), 0, (hipStream_t)stream, d_out, vocab, ld,
                       (uint64_t)seed, slope, noise);
    LAL_HIP(hipGetLastError());
    return LAL_GPU_OK;
}

int lal_gpu_synth_bits(uint32_t *d_out, int batch, int vocab, int words_ld, unsigned long long seed,
                       float p_one, void *stream)
{
    if (!d_out || batch <= 0 || vocab <= 0 || words_ld < (vocab + 31) / 32) return LAL_GPU_E_INVAL;
    const dim3 grid((words_ld + 255) / 256, batch);
    hipLaunchKernelGGL(synth_bits_kernel, grid, dim3(256), 0, (hipStream_t)stream, d_out, vocab,
                       words_ld, (uint64_t)seed, p_one);
    LAL_HIP(hipGetLastError());
    return LAL_GPU_OK;
}

int lal_gpu_synth_int8(int8_t *d_out, size_t n, unsigned long long seed, int lo, int hi, void *stream)
{
    if (!d_out || lo > hi || lo < -128 || hi > 127) return LAL_GPU_E_INVAL;
    hipLaunchKernelGGL(synth_int8_kernel, grid_for(n), dim3(256), 0, (hipStream_t)stream, d_out, n,
                       (uint64_t)seed, lo, hi);
    LAL_HIP(hipGetLastError());
    return LAL_GPU_OK;
}

int lal_gpu_synth_uniform(float *d_out, size_t n, unsigned long long seed, float lo, float hi, void *stream)
{
    if (!d_out) return LAL_GPU_E_INVAL;
    hipLaunchKernelGGL(synth_uniform_kernel, grid_for(n), dim3(256), 0, (hipStream_t)stream, d_out, n,
                       (uint64_t)seed, lo, hi);
    LAL_HIP(hipGetLastError());
    return LAL_GPU_OK;
}

int lal_gpu_synth_normal(float *d_out, size_t n, unsigned long long seed, float sigma, void *stream)
{
    if (!d_out) return LAL_GPU_E_INVAL;
    hipLaunchKernelGGL(synth_normal_kernel, grid_for(n), dim3(256), 0, (hipStream_t)stream, d_out, n,
                       (uint64_t)seed, sigma);
    LAL_HIP(hipGetLastError());
    return LAL_GPU_OK;
}

int lal_gpu_synth_ids(int *d_out, size_t n, unsigned long long seed, int vocab, void *stream)
{
    if (!d_out || vocab <= 0) return LAL_GPU_E_INVAL;
    hipLaunchKernelGGL(synth_ids_kernel, grid_for(n), dim3(256), 0, (hipStream_t)stream, d_out, n,
                       (uint64_t)seed, vocab);
    LAL_HIP(hipGetLastError());
    return LAL_GPU_OK;
}

int lal_gpu_copy(void *d_dst, const void *d_src, size_t bytes, void *stream)
{
    if (!d_dst || !d_src || (bytes & 15) || ((uintptr_t)d_dst & 15) || ((uintptr_t)d_src & 15))
        return LAL_GPU_E_INVAL;
    const size_t n4 = bytes / 16;
    if (n4 == 0) return LAL_GPU_OK;
    size_t blocks = (n4 + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(copy_f32x4_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       (f32x4 *)d_dst, (const f32x4 *)d_src, n4);
    LAL_HIP(hipGetLastError());
    return LAL_GPU_OK;
}

// Test hook: order-insensitive hash of glibc-restated expf over the inputs
// [hi<<16, (hi+1)<<16) for hi in [first_hi, first_hi+nhi), one uint64 each.
int lal_gpu_expf_check(unsigned first_hi, int nhi, unsigned long long *d_out, void *stream)
{
    if (!d_out || nhi <= 0 || first_hi + (unsigned)nhi > 65536u) return LAL_GPU_E_INVAL;
    hipLaunchKernelGGL(expf_check_kernel, dim3(nhi), dim3(256), 0, (hipStream_t)stream, first_hi, nhi,
                       (uint64_t *)d_out);
    LAL_HIP(hipGetLastError());
    return LAL_GPU_OK;
}

}  // extern "C"
