// sample.hip -- the sampler on the device (reference: sampler/sampler.odin:
// 68-199, without the JSON grammar mask), so a sampled decode loop needs no
// logits on the host.
//
// A draw is a short sequence of launches over G workgroups, each owning a
// contiguous slice of SLICE = 2048 logits (75 workgroups at the Qwen3
// vocabulary), so every pass over the vocabulary is spread over the chip
// instead of one CU (one workgroup reads the 600 KB of logits, written by the
// vocabulary GEMV on all eight XCDs, at ~25 GB/s).  Values that one launch
// hands to the next (per-workgroup partials, histograms, the selection in
// progress) live in a SampleWork record in device memory.  Steps, in the
// reference's order:
//   1. repetition penalty on each distinct recent token (positive logits
//      divided, others multiplied), sampler.odin:142-160;
//   2. temperature 0: first maximum (sample_argmax :79-89); otherwise
//      x / temperature, softmax (max, exp(x - max), sum, divide; ops.odin
//      :21-37), one xorshift draw (random_u32 / random_f32 :68-77);
//   3. top-p outside (0, 1): the first index whose running probability
//      exceeds the coin (sample_mult :91-100); inside: candidates p >=
//      (1 - topp) / (n - 1), ordered by p descending (ties: lower index
//      first), cut after the first prefix whose mass exceeds topp, and the
//      coin times that mass located in the same order (sample_topp :106-139).
// Running masses are exact: each probability is taken as a 64-bit fixed-point
// number (p * 2^40, rounded) and summed in integers, so the result does not
// depend on the summation order (the reference's sequential f32 sums carry
// ~1e-5 of rounding over 150k terms; picks can differ from it only when the
// target lies within that rounding of a boundary).  The softmax sum is an f32
// sum in a fixed order (per workgroup of exp(x - the workgroup's maximum),
// then the workgroups in order, each rescaled by exp(its maximum - the
// maximum): one pass for the maximum and the sum), the same in every
// workgroup that needs it.  The top-p order is never
// materialised: the boundary element is found by radix selection over the
// float bits of p (positive floats order as their bit patterns; the sign bit
// is 0), three digits from the top (bits 30..20, 19..9, 8..0: 2048, 2048 and
// 512 buckets), one launch per digit, each workgroup adding its candidates'
// per-bucket count, mass and lowest index to a device histogram and every
// workgroup walking the previous digit's histogram the same way (four 8-bit
// digits took two launches more per draw: 63.5 us against ~50).
//
// Launches per draw: temperature 0: 2; multinomial: 3; top-p: 8.  The
// sequence depends only on the mode (sample_mode), which the caller knows,
// so a captured graph holds one mode's sequence.

#include "device_common.h"

namespace oi {

namespace {

constexpr int SB = 256, SBW = SB / WAVE;   // threads per workgroup, waves
constexpr int SLICE = 2048;                // logits per workgroup: two blocks of 4 per thread
constexpr int SAMPLE_MAX_VOCAB = 1 << 18;
constexpr int MAXG = SAMPLE_MAX_VOCAB / SLICE;

// p * 2^40 rounded to the nearest integer (the scaling is exact in f32, rintf
// rounds the fraction), so the fixed-point total is unbiased against the f32 sum
__device__ __forceinline__ uint64_t fix40(float p) { return (uint64_t)rintf(p * 1099511627776.0f); }

constexpr int NB = 2048;  // buckets of a digit
// digit t from the top: bits [SH[t], SH[t] + WD[t])
__device__ __forceinline__ int dshift(int t) { return t == 0 ? 20 : t == 1 ? 9 : 0; }
__device__ __forceinline__ uint32_t dmask(int t) { return t == 2 ? 511u : 2047u; }
struct Hist {
    uint32_t cnt[NB];
    uint32_t lo[NB];  // lowest index in the bucket
    unsigned long long mass[NB];
};

// The selection in progress, handed from one digit's launch to the next
// (stage k reads slot k and writes slot k + 1, so no launch overwrites what
// another workgroup of the same launch still has to read).
struct Sel {
    uint32_t prefix, mask, tie_lo, tie_cnt;
    unsigned long long above, target, c1;
    int32_t all, done, pad0, pad1;  // all: the candidates' whole mass within topp; done: pick made
};

constexpr int NHIST = 5;  // digit histograms: boundary digits 0..2 -> 0..2, coin digits 1, 2 -> 3, 4
constexpr int NSEL = 8;
struct SampleWork {
    Hist h[NHIST];
    float pmax[MAXG], psum[MAXG];
    int32_t pidx[MAXG];
    uint32_t pties[MAXG];
    unsigned long long pmass[MAXG];
    Sel sel[NSEL];
    uint32_t coin_k;
};

__host__ __device__ __forceinline__ int wg_count(int n) { return (n + SLICE - 1) / SLICE; }

// The thread's elements: block k (0, 1) holds base + 1024 k + 4 tid + x, so
// in index order a workgroup's elements are block 0 by thread, then block 1.
__device__ __forceinline__ int elem(int base, int k, int x) { return base + 1024 * k + 4 * (int)threadIdx.x + x; }

__device__ __forceinline__ void load8(const float *src, int base, int n, float (&v)[2][4]) {
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int i = elem(base, k, 0);
        if (i + 3 < n) {
            const float4 q = *(const float4 *)(src + i);
            v[k][0] = q.x;
            v[k][1] = q.y;
            v[k][2] = q.z;
            v[k][3] = q.w;
        } else {
#pragma unroll
            for (int x = 0; x < 4; x++) v[k][x] = i + x < n ? src[i + x] : 0.f;
        }
    }
}
__device__ __forceinline__ void store8(float *dst, int base, int n, const float (&v)[2][4]) {
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int i = elem(base, k, 0);
        if (i + 3 < n) *(float4 *)(dst + i) = float4{v[k][0], v[k][1], v[k][2], v[k][3]};
        else
#pragma unroll
            for (int x = 0; x < 4; x++)
                if (i + x < n) dst[i + x] = v[k][x];
    }
}

struct Lds {
    Hist h;
    float fv[SBW];
    int iv[SBW];
    unsigned long long uv[SBW];
    uint32_t pen_bits[SLICE / 32];
    int pen_tok[SAMPLE_WINDOW];
    float pen_val[SAMPLE_WINDOW];
    int n_pen, pick;
    Sel s;
};

// (value, index) maximum with the lower index on ties; NaN never wins
__device__ __forceinline__ void argmax_combine(float &v, int &i, float ov, int oi) {
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}
__device__ void block_argmax(float &v, int &i, Lds &s) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) argmax_combine(v, i, __shfl_xor(v, o, WAVE), __shfl_xor(i, o, WAVE));
    if ((threadIdx.x & (WAVE - 1)) == 0) {
        s.fv[threadIdx.x / WAVE] = v;
        s.iv[threadIdx.x / WAVE] = i;
    }
    __syncthreads();
    v = s.fv[0];
    i = s.iv[0];
    for (int w = 1; w < SBW; w++) argmax_combine(v, i, s.fv[w], s.iv[w]);
    __syncthreads();
}
// f32 sum in a fixed order: the thread's own elements in order, lanes by a
// butterfly, waves in order
__device__ float block_sum(float v, Lds &s) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    if ((threadIdx.x & (WAVE - 1)) == 0) s.fv[threadIdx.x / WAVE] = v;
    __syncthreads();
    float r = 0.f;
    for (int w = 0; w < SBW; w++) r += s.fv[w];
    __syncthreads();
    return r;
}
__device__ unsigned long long block_sum_u64(unsigned long long v, Lds &s) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    if ((threadIdx.x & (WAVE - 1)) == 0) s.uv[threadIdx.x / WAVE] = v;
    __syncthreads();
    unsigned long long r = 0;
    for (int w = 0; w < SBW; w++) r += s.uv[w];
    __syncthreads();
    return r;
}
// exclusive prefix over the threads in thread order (and the total)
__device__ unsigned long long block_excl_scan(unsigned long long v, Lds &s, unsigned long long *total) {
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    unsigned long long incl = v;
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
        const unsigned long long y = __shfl_up(incl, o, WAVE);
        if (lane >= o) incl += y;
    }
    if (lane == WAVE - 1) s.uv[w] = incl;
    __syncthreads();
    unsigned long long before = 0, tot = 0;
    for (int i = 0; i < SBW; i++) {
        if (i < w) before += s.uv[i];
        tot += s.uv[i];
    }
    __syncthreads();
    *total = tot;
    return before + incl - v;
}

// The first element of the workgroup's slice, in index order, at which
// carry + running weight exceeds target (weights wt[k][x] of the thread's
// elements); -1 if none.  Every thread gets the result.
__device__ int block_find(const unsigned long long (&wt)[2][4], int base, unsigned long long carry,
                          unsigned long long target, Lds &s) {
    if (threadIdx.x == 0) s.pick = -1;
    __syncthreads();
    for (int k = 0; k < 2; k++) {
        const unsigned long long mine = wt[k][0] + wt[k][1] + wt[k][2] + wt[k][3];
        unsigned long long tot;
        const unsigned long long before = block_excl_scan(mine, s, &tot);
        if (carry + before <= target && target < carry + before + mine) {  // exactly one thread
            unsigned long long run = carry + before;
            for (int x = 0; x < 4; x++) {
                run += wt[k][x];
                if (run > target) {
                    s.pick = elem(base, k, x);
                    break;
                }
            }
        }
        __syncthreads();
        if (s.pick >= 0) break;
        carry += tot;
    }
    const int r = s.pick;
    __syncthreads();
    return r;
}

// Bucket of h where the running mass from the top, starting at *above, first
// exceeds target; -1 if none.  *above becomes the mass of the higher buckets.
// Thread t takes buckets NB-1-8t .. NB-8-8t (descending); the crossing thread
// walks its eight; the result goes to every thread.
__device__ int walk_buckets(const Hist &h, unsigned long long target, unsigned long long *above, Lds &s) {
    constexpr int BPT = NB / SB;
    unsigned long long m[BPT], sum = 0;
#pragma unroll
    for (int x = 0; x < BPT; x++) {
        m[x] = h.mass[NB - 1 - BPT * (int)threadIdx.x - x];
        sum += m[x];
    }
    if (threadIdx.x == 0) s.pick = -1;
    unsigned long long tot;
    const unsigned long long base = *above + block_excl_scan(sum, s, &tot);  // (its barriers order s.pick)
    if (base <= target && target < base + sum) {  // exactly one thread
        unsigned long long run = base;
        int sel = -1;
        for (int x = 0; x < BPT; x++) {
            if (run + m[x] > target) {
                sel = NB - 1 - BPT * (int)threadIdx.x - x;
                break;
            }
            run += m[x];
        }
        s.pick = sel;
        s.s.above = run;
    }
    __syncthreads();
    const int sel = s.pick;
    *above = sel >= 0 ? s.s.above : *above + tot;
    __syncthreads();
    return sel;
}

// A thread's run of equal buckets, added to LDS when the bucket changes
// (flat distributions put most elements of a slice in one bucket).
struct Run {
    int b = -1;
    uint32_t c = 0, lo = 0;
    uint64_t m = 0;
    __device__ void flush(Hist &h) {
        if (b < 0) return;
        atomicAdd(&h.cnt[b], c);
        atomicAdd(&h.mass[b], (unsigned long long)m);
        atomicMin(&h.lo[b], lo);
    }
    __device__ void add(Hist &h, int bucket, int i, uint64_t mass) {
        if (bucket != b) {
            flush(h);
            b = bucket;
            c = 0;
            m = 0;
            lo = (uint32_t)i;  // a thread's elements come in increasing index order
        }
        c++;
        m += mass;
    }
};

// (cnt_lo false: the masses only, the histogram of a digit whose counts and
// lowest indices are not flushed)
__device__ void hist_clear(Hist &h, bool cnt_lo) {
    for (int i = threadIdx.x; i < NB; i += SB) {
        if (cnt_lo) {
            h.cnt[i] = 0;
            h.lo[i] = 0xFFFFFFFFu;
        }
        h.mass[i] = 0;
    }
}

// The workgroup's histogram added to the device histogram: the masses always
// (a candidate's fix40 mass is > 0), the counts and lowest indices only for
// the last digit, the only one whose are read (the pick's equal
// probabilities); every atomic is one more on an address that all 75
// workgroups update, so the first digits' histograms cost a third of it.
__device__ void hist_flush(const Hist &h, Hist *g, bool cnt_lo) {
    for (int b = threadIdx.x; b < NB; b += SB)
        if (h.mass[b]) {
            atomicAdd(&g->mass[b], h.mass[b]);
            if (cnt_lo) {
                atomicAdd(&g->cnt[b], h.cnt[b]);
                atomicMin(&g->lo[b], h.lo[b]);
            }
        }
}

// digit t histogram of the slice's candidates whose bits match prefix under
// mask, added to the device histogram g
__device__ void hist_digit(const float *p, int base, int n, float cutoff, int t, uint32_t prefix, uint32_t mask,
                           Hist *g, Lds &s) {
    hist_clear(s.h, t == 2);
    float v[2][4];
    load8(p, base, n, v);
    __syncthreads();
    Run run;
#pragma unroll
    for (int k = 0; k < 2; k++)
#pragma unroll
        for (int x = 0; x < 4; x++) {
            const int i = elem(base, k, x);
            const uint32_t key = __float_as_uint(v[k][x]);
            if (i < n && v[k][x] >= cutoff && (key & mask) == prefix)
                run.add(s.h, (int)((key >> dshift(t)) & dmask(t)), i, fix40(v[k][x]));
        }
    run.flush(s.h);
    __syncthreads();
    hist_flush(s.h, g, t == 2);
}

__device__ __forceinline__ float cutoff_of(const SampleState *ss, int n) {
    return (1.0f - ss->topp) / (float)(n - 1);
}

// The pick: record_token (sampler.odin:50-56) and the token loop's state.
// One thread.
__device__ void finalize(int pick, SampleState *ss, int32_t *state, int32_t *tokens_out, int32_t *pick_out) {
    const float pen = ss->penalty < 1.0f ? 1.0f : ss->penalty;
    if (ss->record && pen != 1.0f) {
        int nl = min(ss->n_last, SAMPLE_WINDOW);
        if (nl == SAMPLE_WINDOW) {
            for (int i = 1; i < SAMPLE_WINDOW; i++) ss->last[i - 1] = ss->last[i];
            nl--;
        }
        ss->last[nl] = pick;
        ss->n_last = nl + 1;
    }
    if (state) {  // advance the token loop as the greedy reduction does
        const int step = state[ST_STEP];
        if (tokens_out && step >= 0 && step < state[ST_CAP]) tokens_out[step] = pick;
        state[ST_STEP] = step + 1;
        state[ST_TOKEN] = pick;
        state[ST_POS] = state[ST_POS] + 1;
        state[ST_PENDING] = 0;
    }
    if (pick_out) *pick_out = pick;
}

struct SArgs {
    const float *logits;
    float *p;
    int n;
    SampleState *ss;
    SampleWork *w;
    int32_t *state, *tokens_out, *pick_out;
};

// 1. Penalty (distinct recent tokens, each once) and temperature into p; the
// slice's first maximum.  Workgroup 0 also clears the digit histograms.
__global__ __launch_bounds__(SB) void sample_penalty_kernel(SArgs a) {
#pragma clang fp contract(off)
    __shared__ Lds s;
    const int base = blockIdx.x * SLICE, tid = threadIdx.x;
    const SampleState *ss = a.ss;
    // enable_repeat_penalty's clamp (sampler.odin:42-44) applied here too, so a
    // C caller's penalty below 1 acts as 1 (off) rather than dividing by it
    const float T = ss->temperature, pen = ss->penalty < 1.0f ? 1.0f : ss->penalty;
    {  // the digit histograms, cleared by all workgroups (bucket i of every histogram by one thread)
        const int G = wg_count(a.n);
        for (int i = blockIdx.x * SB + tid; i < NHIST * NB; i += G * SB) {
            Hist &h = a.w->h[i / NB];
            h.cnt[i % NB] = 0;
            h.lo[i % NB] = 0xFFFFFFFFu;
            h.mass[i % NB] = 0;
        }
    }
    for (int i = tid; i < SLICE / 32; i += SB) s.pen_bits[i] = 0;
    if (tid == 0) s.n_pen = 0;
    __syncthreads();
    const int nl = min(ss->n_last, SAMPLE_WINDOW);
    if (pen != 1.0f && tid < nl) {
        const int tok = ss->last[tid];
        bool dup = false;
        for (int j = 0; j < tid; j++) dup |= ss->last[j] == tok;
        if (!dup && tok >= base && tok < base + SLICE && tok < a.n) {
            const float v = a.logits[tok];
            const int slot = atomicAdd(&s.n_pen, 1);
            s.pen_tok[slot] = tok;
            s.pen_val[slot] = v > 0.f ? v / pen : v * pen;
            atomicOr(&s.pen_bits[(tok - base) >> 5], 1u << ((tok - base) & 31));
        }
    }
    __syncthreads();
    float v[2][4];
    load8(a.logits, base, a.n, v);
    const bool greedy = T == 0.0f;
    float m = -INFINITY;
    int mi = 0x7FFFFFFF;
#pragma unroll
    for (int k = 0; k < 2; k++)
#pragma unroll
        for (int x = 0; x < 4; x++) {
            const int i = elem(base, k, x);
            if (i >= a.n) continue;
            float x0 = v[k][x];
            if (s.pen_bits[(i - base) >> 5] & (1u << ((i - base) & 31)))
                for (int q = 0; q < s.n_pen; q++)
                    if (s.pen_tok[q] == i) x0 = s.pen_val[q];
            if (!greedy) x0 = x0 / T;
            v[k][x] = x0;
            argmax_combine(m, mi, x0, i);
        }
    store8(a.p, base, a.n, v);
    block_argmax(m, mi, s);
    // the slice's sum of exp(x - its maximum), for the softmax's sum
    float sum = 0.f;
    if (!greedy && m != -INFINITY) {
#pragma unroll
        for (int k = 0; k < 2; k++)
#pragma unroll
            for (int x = 0; x < 4; x++)
                if (elem(base, k, x) < a.n) sum += expf(v[k][x] - m);
    }
    sum = block_sum(sum, s);
    if (tid == 0) {
        a.w->pmax[blockIdx.x] = m;
        a.w->pidx[blockIdx.x] = mi;
        a.w->psum[blockIdx.x] = sum;
    }
}

// 2. The maximum over the slices.  Temperature 0: workgroup 0 picks it.
// Otherwise p = exp(x - max) / sum, the sum over the slices in order of each
// slice's sum rescaled to the maximum (sum_g s_g exp(m_g - max), so the
// maximum and the sum take one pass), then the slice's fixed-point mass
// (multinomial) or its candidates' first-digit histogram (top-p).  Workgroup
// 0 draws the coin (random_f32, sampler.odin:68-77).
__global__ __launch_bounds__(SB) void sample_norm_kernel(SArgs a, int mode) {
#pragma clang fp contract(off)
    __shared__ Lds s;
    const int G = wg_count(a.n), base = blockIdx.x * SLICE, tid = threadIdx.x;
    // the slices' partials, one per thread (G <= 128 <= SB), requested
    // together: a loop over them in one thread waited for each in turn
    const float pm = tid < G ? a.w->pmax[tid] : -INFINITY, ps = tid < G ? a.w->psum[tid] : 0.f;
    float mx = pm;
    int mi = tid < G ? a.w->pidx[tid] : 0x7FFFFFFF;
    block_argmax(mx, mi, s);
    if (mode == SAMPLE_GREEDY) {
        if (blockIdx.x == 0 && threadIdx.x == 0)
            finalize(mi == 0x7FFFFFFF ? 0 : mi, a.ss, a.state, a.tokens_out, a.pick_out);
        return;
    }
    const bool topp_mode = mode == SAMPLE_TOPP;
    const float tot = block_sum(pm != -INFINITY ? ps * expf(pm - mx) : 0.f, s);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        uint64_t x = a.ss->rng;
        x ^= x >> 12;
        x ^= x << 25;
        x ^= x >> 27;
        a.ss->rng = x;
        a.w->coin_k = (uint32_t)((x * 0x2545F4914F6CDD1Dull) >> 32) >> 8;  // coin = coin_k / 2^24
    }
    float v[2][4];
    load8(a.p, base, a.n, v);
#pragma unroll
    for (int k = 0; k < 2; k++)
#pragma unroll
        for (int x = 0; x < 4; x++) v[k][x] = expf(v[k][x] - mx) / tot;
    store8(a.p, base, a.n, v);
    if (!topp_mode) {
        unsigned long long m = 0;
#pragma unroll
        for (int k = 0; k < 2; k++)
#pragma unroll
            for (int x = 0; x < 4; x++)
                if (elem(base, k, x) < a.n) m += fix40(v[k][x]);
        m = block_sum_u64(m, s);
        if (threadIdx.x == 0) a.w->pmass[blockIdx.x] = m;
        return;
    }
    const float cutoff = cutoff_of(a.ss, a.n);
    hist_clear(s.h, false);
    __syncthreads();
    Run run;
#pragma unroll
    for (int k = 0; k < 2; k++)
#pragma unroll
        for (int x = 0; x < 4; x++) {
            const int i = elem(base, k, x);
            if (i < a.n && v[k][x] >= cutoff)
                run.add(s.h, (int)((__float_as_uint(v[k][x]) >> dshift(0)) & dmask(0)), i, fix40(v[k][x]));
        }
    run.flush(s.h);
    __syncthreads();
    hist_flush(s.h, &a.w->h[0], false);
}

// 4 (multinomial, sample_mult): the first index whose running mass exceeds
// the coin; the last index when none does.
__global__ __launch_bounds__(SB) void sample_mult_kernel(SArgs a) {
    __shared__ Lds s;
    const int G = wg_count(a.n), base = blockIdx.x * SLICE, tid = threadIdx.x;
    const unsigned long long pg = tid < G ? a.w->pmass[tid] : 0;  // one slice's mass per thread
    const unsigned long long before = block_sum_u64(tid < (int)blockIdx.x ? pg : 0, s), total = block_sum_u64(pg, s);
    const unsigned long long target = (unsigned long long)a.w->coin_k << 16;  // coin * 2^40, exact
    if (total <= target) {
        if (blockIdx.x == 0 && threadIdx.x == 0) finalize(a.n - 1, a.ss, a.state, a.tokens_out, a.pick_out);
        return;
    }
    if (!(before <= target && target < before + a.w->pmass[blockIdx.x])) return;
    float v[2][4];
    load8(a.p, base, a.n, v);
    unsigned long long wt[2][4];
#pragma unroll
    for (int k = 0; k < 2; k++)
#pragma unroll
        for (int x = 0; x < 4; x++) wt[k][x] = elem(base, k, x) < a.n ? fix40(v[k][x]) : 0;
    const int f = block_find(wt, base, before, target, s);
    if (threadIdx.x == 0) finalize(f < 0 ? a.n - 1 : f, a.ss, a.state, a.tokens_out, a.pick_out);
}

// Top-p digit rounds.  Stage k (0-based) reads a.w->sel[k] (stage 0: none)
// and writes sel[k + 1]:
//   stage 0: boundary target fix40(topp): walk digit 0 (h[0]), histogram digit 1 -> h[1]
//   stage 1: walk h[1], histogram digit 2 -> h[2]
//   stage 2: walk h[2] -> the boundary value; c1 = the mass through it; coin
//            target r = coin * c1: walk h[0] again, histogram digit 1 -> h[3]
//   stage 3: walk h[3], histogram digit 2 -> h[4]
//   stage 4: walk h[4] -> the pick value; if its rank among equal
//            probabilities is 0 (or it has no equal), the pick; otherwise
//            each slice counts its equal elements
//   stage 5: the slice holding that rank finds it
__global__ __launch_bounds__(SB) void sample_topp_kernel(SArgs a, int stage) {
    __shared__ Lds s;
    const int base = blockIdx.x * SLICE, tid = threadIdx.x;
    const float cutoff = cutoff_of(a.ss, a.n);
    SampleWork *w = a.w;
    Sel cur;
    if (stage == 0) {
        cur = Sel{};
        cur.target = fix40(a.ss->topp);
    } else {
        cur = w->sel[stage];
    }
    if (cur.done) {  // the pick is made: later stages pass it on
        if (blockIdx.x == 0 && tid == 0) w->sel[stage + 1] = cur;
        return;
    }
    auto walk_digit = [&](const Hist &gh, int t) -> int {
        unsigned long long above = cur.above;
        const int sel = walk_buckets(gh, cur.target, &above, s);
        if (sel >= 0) {
            cur.above = above;
            cur.prefix |= (uint32_t)sel << dshift(t);
            cur.mask |= dmask(t) << dshift(t);
            cur.tie_lo = gh.lo[sel];
            cur.tie_cnt = gh.cnt[sel];
        }
        return sel;
    };
    if (stage == 0 || stage == 1 || stage == 3) {
        const int hin = stage == 0 ? 0 : stage, t = stage == 3 ? 1 : stage;  // histogram and digit walked
        const int sel = cur.all ? -1 : walk_digit(w->h[hin], t);
        if (sel < 0) {
            // boundary: the candidates' whole mass is within topp, so all of
            // them are kept (the coin stage then takes c1 = that mass);
            // coin: unreachable (r < c1), pick 0 as the reference's fallback
            if (stage < 2) cur.all = 1;
            else {
                cur.done = 1;
                if (blockIdx.x == 0 && tid == 0) finalize(0, a.ss, a.state, a.tokens_out, a.pick_out);
            }
        } else {
            hist_digit(a.p, base, a.n, cutoff, t + 1, cur.prefix, cur.mask, &w->h[stage == 3 ? 4 : hin + 1], s);
        }
        if (blockIdx.x == 0 && tid == 0) w->sel[stage + 1] = cur;
        return;
    }
    if (stage == 2) {
        if (!cur.all) {
            walk_digit(w->h[2], 2);
            // equal probabilities in index order: the j-th crosses
            const uint64_t P = fix40(__uint_as_float(cur.prefix));
            const uint64_t j = P ? (cur.target - cur.above) / P : 0;
            cur.c1 = cur.above + (j + 1) * P;
        } else {
            unsigned long long t = 0;
            for (int b = tid; b < NB; b += SB) t += w->h[0].mass[b];
            cur.c1 = block_sum_u64(t, s);
        }
        // r = coin * c1: (c1 * coin_k) >> 24 without overflow
        const unsigned long long ck = w->coin_k, lo = cur.c1 * ck, hi = __umul64hi(cur.c1, ck);
        Sel nxt{};
        nxt.target = (hi << 40) | (lo >> 24);
        cur = nxt;
        const int sel = walk_digit(w->h[0], 0);
        if (sel < 0) {  // unreachable: r < c1
            cur.done = 1;
            if (blockIdx.x == 0 && tid == 0) finalize(0, a.ss, a.state, a.tokens_out, a.pick_out);
        } else {
            hist_digit(a.p, base, a.n, cutoff, 1, cur.prefix, cur.mask, &w->h[3], s);
        }
        if (blockIdx.x == 0 && tid == 0) w->sel[stage + 1] = cur;
        return;
    }
    if (stage == 4) {
        const int sel = walk_digit(w->h[4], 2);
        if (sel < 0) {  // unreachable
            cur.done = 1;
            if (blockIdx.x == 0 && tid == 0) finalize(0, a.ss, a.state, a.tokens_out, a.pick_out);
            if (blockIdx.x == 0 && tid == 0) w->sel[stage + 1] = cur;
            return;
        }
        const uint64_t P = fix40(__uint_as_float(cur.prefix));
        const uint64_t j = P ? (cur.target - cur.above) / P : 0;
        if (j == 0 || cur.tie_cnt <= 1) {
            cur.done = 1;
            if (blockIdx.x == 0 && tid == 0) finalize((int)cur.tie_lo, a.ss, a.state, a.tokens_out, a.pick_out);
        } else {
            cur.c1 = j;  // the rank, for stage 5
            float v[2][4];
            load8(a.p, base, a.n, v);
            unsigned long long c = 0;
#pragma unroll
            for (int k = 0; k < 2; k++)
#pragma unroll
                for (int x = 0; x < 4; x++) c += elem(base, k, x) < a.n && __float_as_uint(v[k][x]) == cur.prefix;
            c = block_sum_u64(c, s);
            if (tid == 0) w->pties[blockIdx.x] = (uint32_t)c;
        }
        if (blockIdx.x == 0 && tid == 0) w->sel[stage + 1] = cur;
        return;
    }
    // stage 5: rank j among the equal probabilities, in index order
    const unsigned long long before =
        block_sum_u64(tid < (int)blockIdx.x && tid < wg_count(a.n) ? w->pties[tid] : 0u, s);
    const unsigned long long j = cur.c1;
    if (!(before <= j && j < before + w->pties[blockIdx.x])) return;
    float v[2][4];
    load8(a.p, base, a.n, v);
    unsigned long long wt[2][4];
#pragma unroll
    for (int k = 0; k < 2; k++)
#pragma unroll
        for (int x = 0; x < 4; x++) wt[k][x] = elem(base, k, x) < a.n && __float_as_uint(v[k][x]) == cur.prefix;
    const int f = block_find(wt, base, before, j, s);
    if (tid == 0) finalize(f < 0 ? (int)cur.tie_lo : f, a.ss, a.state, a.tokens_out, a.pick_out);
}

}  // namespace

int sample_max_vocab() { return SAMPLE_MAX_VOCAB; }
size_t sample_work_bytes() { return sizeof(SampleWork); }
int sample_mode(float temperature, float topp, int n) {
    if (temperature == 0.0f) return SAMPLE_GREEDY;
    return !(topp > 0.f && topp < 1.f) || n == 1 ? SAMPLE_MULT : SAMPLE_TOPP;
}

hipError_t launch_sample(const float *logits, float *p, int n, SampleState *ss, int mode, void *work, int32_t *state,
                         int32_t *tokens_out, int32_t *pick, hipStream_t st) {
    if (n <= 0 || n > SAMPLE_MAX_VOCAB || !work || mode < SAMPLE_GREEDY || mode > SAMPLE_TOPP)
        return hipErrorInvalidValue;
    const SArgs a{logits, p, n, ss, (SampleWork *)work, state, tokens_out, pick};
    const dim3 grid((unsigned)wg_count(n));
    hipLaunchKernelGGL(sample_penalty_kernel, grid, dim3(SB), 0, st, a);
    hipLaunchKernelGGL(sample_norm_kernel, grid, dim3(SB), 0, st, a, mode);
    if (mode == SAMPLE_GREEDY) return hipGetLastError();
    if (mode == SAMPLE_MULT) {
        hipLaunchKernelGGL(sample_mult_kernel, grid, dim3(SB), 0, st, a);
        return hipGetLastError();
    }
    for (int stage = 0; stage < 6; stage++) hipLaunchKernelGGL(sample_topp_kernel, grid, dim3(SB), 0, st, a, stage);
    return hipGetLastError();
}

}  // namespace oi
