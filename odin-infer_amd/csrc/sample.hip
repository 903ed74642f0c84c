// sample.hip -- the sampler on the device (reference: sampler/sampler.odin:
// 68-199, without the JSON grammar mask), so a sampled decode loop needs no
// logits on the host.
//
// One workgroup of 1024 threads (16 waves) per draw.  Wave w owns the index
// range [w*W, (w+1)*W) (W a multiple of 1024) and walks it 1024 elements at a
// time, each lane loading four 16-byte groups, so every pass is coalesced and
// per-wave totals come in index order.  (One workgroup streams the 600 KB of
// a 150k vocabulary at ~25 GB/s -- the logits come from the other XCDs' L2
// through the MALL -- so a draw costs 50 us at temperature 0 and ~400 us with
// top-p on the Qwen3 vocabulary.)  Steps, in the reference's order:
//   1. repetition penalty on each distinct recent token (positive logits
//      divided, others multiplied), sampler.odin:142-160 -- the tokens are
//      marked in an LDS bitmap so the pass over the logits stays one read;
//   2. temperature 0: first maximum (sample_argmax :79-89); otherwise
//      x / temperature, softmax (max, exp(x - max), sum, divide; ops.odin
//      :21-37), one xorshift draw (random_u32 / random_f32 :68-77);
//   3. top-p outside (0, 1): the first index whose running probability
//      exceeds the coin (sample_mult :91-100); inside: candidates p >=
//      (1 - topp) / (n - 1), ordered by p descending (ties: lower index
//      first), cut after the first prefix whose mass exceeds topp, and the
//      coin times that mass located in the same order (sample_topp :106-139).
// Running masses are exact: each probability is taken as a 64-bit fixed-point
// number (p * 2^40, truncated) and summed in integers, so the result does not
// depend on the summation order (the reference's sequential f32 sums carry
// ~1e-5 of rounding over 150k terms; picks can differ from it only when the
// target lies within that rounding of a boundary).  The top-p order is never
// materialised: the boundary element is found by radix selection over the
// float bits of p (positive floats order as their bit patterns), four 8-bit
// digits from the top, with per-bucket count, mass and lowest index in LDS.
// A lane adds runs of equal buckets before touching LDS, so the flat
// distributions that put most elements in one bucket do not serialise on one
// address.  The first digit's histogram is shared by both selections.

#include "device_common.h"

namespace oi {

namespace {

constexpr int SWG = 1024, SWAVES = SWG / WAVE;
constexpr int SAMPLE_MAX_VOCAB = 1 << 18;  // LDS penalty bitmap: 32 KB

// p * 2^40 rounded to the nearest integer (the scaling is exact in f32, rintf
// rounds the fraction), so the fixed-point total is unbiased against the f32 sum
__device__ __forceinline__ uint64_t fix40(float p) { return (uint64_t)rintf(p * 1099511627776.0f); }

struct Hist {
    uint32_t cnt[256];
    uint32_t lo[256];  // lowest index in the bucket
    unsigned long long mass[256];
};

struct Smem {
    uint32_t pen_bits[SAMPLE_MAX_VOCAB / 32];
    Hist h, h3;  // the current digit's histogram; the first digit's, kept
    uint64_t wtot[SWAVES];
    float fv[SWAVES];
    int iv[SWAVES];
    int pen_tok[SAMPLE_WINDOW];
    float pen_val[SAMPLE_WINDOW];
    uint64_t total, above, u64b;
    int n_pen, sel, pick, ib;
    float fb;
    uint32_t coin_k;
};

// sums over waves in wave order (a wave's value from its lane 0)
__device__ uint64_t waves_excl_scan(uint64_t v, Smem &s, uint64_t *total) {
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    if (lane == 0) s.wtot[w] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t run = 0;
        for (int i = 0; i < SWAVES; i++) {
            const uint64_t t = s.wtot[i];
            s.wtot[i] = run;
            run += t;
        }
        s.total = run;
    }
    __syncthreads();
    const uint64_t r = s.wtot[w];
    if (total) *total = s.total;
    __syncthreads();
    return r;
}

__device__ float wave_max_f(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}

__device__ float block_max(float v, Smem &s) {
    v = wave_max_f(v);
    if ((threadIdx.x & (WAVE - 1)) == 0) s.fv[threadIdx.x / WAVE] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = s.fv[0];
        for (int i = 1; i < SWAVES; i++) m = fmaxf(m, s.fv[i]);
        s.fb = m;
    }
    __syncthreads();
    const float r = s.fb;
    __syncthreads();
    return r;
}

// sum in a fixed order: lanes by a butterfly, waves in order
__device__ float block_sum(float v, Smem &s) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    if ((threadIdx.x & (WAVE - 1)) == 0) s.fv[threadIdx.x / WAVE] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = 0.f;
        for (int i = 0; i < SWAVES; i++) m += s.fv[i];
        s.fb = m;
    }
    __syncthreads();
    const float r = s.fb;
    __syncthreads();
    return r;
}

__device__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

// (value, index) maximum with the lower index on ties; NaN never wins
__device__ int block_argmax(float v, int i, Smem &s) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o, WAVE);
        const int oi = __shfl_xor(i, o, WAVE);
        if (ov > v || (ov == v && oi < i)) {
            v = ov;
            i = oi;
        }
    }
    if ((threadIdx.x & (WAVE - 1)) == 0) {
        s.fv[threadIdx.x / WAVE] = v;
        s.iv[threadIdx.x / WAVE] = i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float bv = s.fv[0];
        int bi = s.iv[0];
        for (int w = 1; w < SWAVES; w++)
            if (s.fv[w] > bv || (s.fv[w] == bv && s.iv[w] < bi)) {
                bv = s.fv[w];
                bi = s.iv[w];
            }
        s.pick = bi == 0x7FFFFFFF ? 0 : bi;
    }
    __syncthreads();
    const int r = s.pick;
    __syncthreads();
    return r;
}

// A lane's run of equal buckets, added to LDS when the bucket changes.
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
            lo = (uint32_t)i;  // elements come in increasing index order per lane
        }
        c++;
        m += mass;
    }
};

__device__ void hist_clear(Hist &h) {
    for (int i = threadIdx.x; i < 256; i += SWG) {
        h.cnt[i] = 0;
        h.lo[i] = 0xFFFFFFFFu;
        h.mass[i] = 0;
    }
}

struct Range {
    int b0, b1;  // this wave's index range
};

// Calls f(i, src[i]) for the wave's range in increasing index order per
// lane.  A lane takes 4 consecutive elements of each 256-element group and
// loads 4 groups (16 values) at once, so 4 16-byte loads are in flight.
constexpr int GROUP = 4 * WAVE, BATCH = 4 * GROUP;

template <class F>
__device__ __forceinline__ void for_each(const float *src, Range r, F f) {
    const int lane = threadIdx.x & (WAVE - 1);
    for (int base = r.b0; base < r.b1; base += BATCH) {
        float v[16];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = base + GROUP * u + 4 * lane;
            if (i + 3 < r.b1) {
                const float4 q = *(const float4 *)(src + i);
                v[4 * u] = q.x;
                v[4 * u + 1] = q.y;
                v[4 * u + 2] = q.z;
                v[4 * u + 3] = q.w;
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++) v[4 * u + k] = i + k < r.b1 ? src[i + k] : 0.f;
            }
        }
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int i = base + GROUP * u + 4 * lane + k;
                if (i < r.b1) f(i, v[4 * u + k]);
            }
    }
}

// digit d histogram of the candidates whose key matches prefix under mask
__device__ void hist_pass(const float *p, Range r, float cutoff, int d, uint32_t prefix, uint32_t mask, Hist &h) {
    Run run;
    for_each(p, r, [&](int i, float v) {
        const uint32_t k = __float_as_uint(v);
        if (v >= cutoff && (k & mask) == prefix) run.add(h, (int)((k >> (8 * d)) & 255u), i, fix40(v));
    });
    run.flush(h);
}

// Index order within a 1024-element batch: group u, lane, element k.  The
// first element of the wave's range, in index order, at which
// carry + running weight(i) exceeds target, where weight(i, v) is given;
// -1 if none.  *carry: the weight before the range on entry.
template <class Wt>
__device__ int wave_find(const float *src, Range r, uint64_t carry, uint64_t target, Wt weight) {
    const int lane = threadIdx.x & (WAVE - 1);
    for (int base = r.b0; base < r.b1; base += GROUP) {
        const int i0 = base + 4 * lane;
        uint64_t wk[4], lsum = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            wk[k] = i0 + k < r.b1 ? weight(i0 + k, src[i0 + k]) : 0;
            lsum += wk[k];
        }
        uint64_t incl = lsum;
#pragma unroll
        for (int o = 1; o < WAVE; o <<= 1) {
            const uint64_t y = __shfl_up(incl, o, WAVE);
            if (lane >= o) incl += y;
        }
        const uint64_t bal = __ballot(carry + incl > target);
        if (bal) {
            const int L = __ffsll((long long)bal) - 1;
            uint64_t run = carry + __shfl(incl - lsum, L, WAVE);
            int found = -1;
            if (lane == L)
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    run += wk[k];
                    if (found < 0 && run > target) found = i0 + k;
                }
            return __shfl(found, L, WAVE);
        }
        carry += __shfl(incl, WAVE - 1, WAVE);
    }
    return -1;
}

// Bucket of digit d (from the top) where the running mass, starting at
// *above, first exceeds target; -1 if none.  *above becomes the mass of the
// higher buckets.  One thread; the result is broadcast through s.
__device__ int walk_buckets(const Hist &h, uint64_t target, uint64_t *above, Smem &s) {
    if (threadIdx.x == 0) {
        uint64_t run = *above;
        int sel = -1;
        for (int b = 255; b >= 0; b--) {
            if (!h.cnt[b]) continue;
            if (run + h.mass[b] > target) {
                sel = b;
                break;
            }
            run += h.mass[b];
        }
        s.sel = sel;
        s.above = run;
    }
    __syncthreads();
    const int sel = s.sel;
    *above = s.above;
    __syncthreads();
    return sel;
}

// The first element, in the order (p descending, index ascending) over the
// candidates p >= cutoff, at which the running mass exceeds `target`; -1 if
// the candidates' whole mass does not.  *through: the running mass including
// that element.  h3: the candidates' first-digit histogram.
__device__ int select_desc(const float *p, Range r, float cutoff, uint64_t target, const Hist &h3, Smem &s,
                           uint64_t *through) {
    const int lane = threadIdx.x & (WAVE - 1);
    uint64_t above = 0;
    int sel = walk_buckets(h3, target, &above, s);
    if (sel < 0) return -1;
    uint32_t prefix = (uint32_t)sel << 24, mask = 0xFF000000u;
    uint32_t tie_lo = h3.lo[sel], tie_cnt = h3.cnt[sel];
    for (int d = 2; d >= 0; d--) {
        hist_clear(s.h);
        __syncthreads();
        hist_pass(p, r, cutoff, d, prefix, mask, s.h);
        __syncthreads();
        sel = walk_buckets(s.h, target, &above, s);
        if (sel < 0) return -1;  // unreachable: the bucket above held the crossing
        prefix |= (uint32_t)sel << (8 * d);
        mask |= 255u << (8 * d);
        tie_lo = s.h.lo[sel];
        tie_cnt = s.h.cnt[sel];
        __syncthreads();
    }
    // equal probabilities in index order: the j-th crosses
    const uint64_t P = fix40(__uint_as_float(prefix));
    const uint64_t j = P ? (target - above) / P : 0;
    *through = above + (j + 1) * P;
    if (j == 0 || tie_cnt <= 1) return (int)tie_lo;
    // rank j among the ties: per-wave counts, then the wave holding it
    uint64_t c = 0;
    for_each(p, r, [&](int, float v) { c += __float_as_uint(v) == prefix; });
    const uint64_t mine = wave_sum_u64(c);
    const uint64_t before = waves_excl_scan(mine, s, nullptr);
    if (before <= j && j < before + mine) {
        const int f = wave_find(p, r, before, j, [&](int, float v) -> uint64_t { return __float_as_uint(v) == prefix; });
        if (lane == 0) s.pick = f;
    }
    __syncthreads();
    const int res = s.pick;
    __syncthreads();
    return res;
}

__global__ __launch_bounds__(SWG) void sample_kernel(const float *logits, float *p, int n, SampleState *ss,
                                                     int32_t *state, int32_t *tokens_out, int32_t *pick_out) {
#pragma clang fp contract(off)
    __shared__ Smem s;
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), w = tid / WAVE;
    const int W = ((n + SWAVES - 1) / SWAVES + BATCH - 1) / BATCH * BATCH;
    const Range r{min(n, w * W), min(n, (w + 1) * W)};
    // enable_repeat_penalty's clamp (sampler.odin:42-44) applied here too, so a
    // C caller's penalty below 1 acts as 1 (off) rather than dividing by it
    const float T = ss->temperature, topp = ss->topp, pen = ss->penalty < 1.0f ? 1.0f : ss->penalty;
    for (int i = tid; i < (n + 31) / 32; i += SWG) s.pen_bits[i] = 0;
    __syncthreads();
    if (tid == 0) {  // distinct recent tokens and their penalised logits
        int np = 0;
        if (pen != 1.0f)
            for (int i = 0; i < ss->n_last && i < SAMPLE_WINDOW; i++) {
                const int tok = ss->last[i];
                if (tok < 0 || tok >= n) continue;
                bool dup = false;
                for (int j = 0; j < np; j++) dup |= s.pen_tok[j] == tok;
                if (dup) continue;
                const float v = logits[tok];
                s.pen_tok[np] = tok;
                s.pen_val[np] = v > 0.f ? v / pen : v * pen;
                s.pen_bits[tok >> 5] |= 1u << (tok & 31);
                np++;
            }
        s.n_pen = np;
        s.pick = 0;
    }
    __syncthreads();
    const bool greedy = T == 0.0f;
    // x = value (/ T) into p; the lane's maximum (first index on ties)
    float m = -INFINITY;
    int mi = 0x7FFFFFFF;
    for_each(logits, r, [&](int i, float v) {
        if (s.pen_bits[i >> 5] & (1u << (i & 31)))
            for (int k = 0; k < s.n_pen; k++)
                if (s.pen_tok[k] == i) v = s.pen_val[k];
        if (!greedy) v = v / T;
        p[i] = v;
        if (v > m) {
            m = v;
            mi = i;
        }
    });
    int pick;
    if (greedy) {
        pick = block_argmax(m, mi, s);
    } else {
        const float mx = block_max(m, s);
        float sum = 0.f;
        for_each(p, r, [&](int i, float x) {
            const float e = expf(x - mx);
            p[i] = e;
            sum += e;
        });
        const float tot = block_sum(sum, s);
        if (tid == 0) {  // random_f32 (sampler.odin:68-77)
            uint64_t x = ss->rng;
            x ^= x >> 12;
            x ^= x << 25;
            x ^= x >> 27;
            ss->rng = x;
            s.coin_k = (uint32_t)((x * 0x2545F4914F6CDD1Dull) >> 32) >> 8;  // coin = coin_k / 2^24
        }
        const bool mult = !(topp > 0.f && topp < 1.f) || n == 1;
        const float cutoff = mult ? 0.f : (1.0f - topp) / (float)(n - 1);
        if (!mult) hist_clear(s.h3);
        __syncthreads();
        const uint64_t coin_k = s.coin_k;
        // p = e / sum; the wave's mass (index order) or the first digit's histogram
        uint64_t wm = 0;
        Run run;
        for_each(p, r, [&](int i, float e) {
            const float q = e / tot;
            p[i] = q;
            if (mult) wm += fix40(q);
            else if (q >= cutoff) run.add(s.h3, (int)(__float_as_uint(q) >> 24), i, fix40(q));
        });
        if (!mult) run.flush(s.h3);
        __syncthreads();
        if (mult) {
            // sample_mult: the first index whose running mass exceeds the coin
            const uint64_t mine = wave_sum_u64(wm);
            const uint64_t before = waves_excl_scan(mine, s, nullptr);
            const uint64_t target = coin_k << 16;  // coin * 2^40, exact
            if (tid == 0) s.pick = n - 1;          // no crossing: the last index
            __syncthreads();
            if (before <= target && target < before + mine) {
                const int f = wave_find(p, r, before, target, [](int, float q) -> uint64_t { return fix40(q); });
                if (lane == 0 && f >= 0) s.pick = f;
            }
            __syncthreads();
            pick = s.pick;
        } else {
            uint64_t c1 = 0;
            const int last = select_desc(p, r, cutoff, fix40(topp), s.h3, s, &c1);
            if (last < 0) {
                // the candidates' whole mass is within topp: all of them
                uint64_t tot3 = 0;
                if (tid == 0)
                    for (int b = 0; b < 256; b++) tot3 += s.h3.mass[b];
                if (tid == 0) s.u64b = tot3;
                __syncthreads();
                c1 = s.u64b;
                __syncthreads();
            }
            // r = coin * cumulative: (c1 * coin_k) >> 24 without overflow
            const uint64_t lo = c1 * coin_k, hi = __umul64hi(c1, coin_k);
            const uint64_t rr = (hi << 40) | (lo >> 24);
            uint64_t dummy;
            pick = select_desc(p, r, cutoff, rr, s.h3, s, &dummy);
            if (pick < 0) pick = 0;  // unreachable: rr < c1
        }
    }
    if (tid == 0) {
        if (ss->record && pen != 1.0f) {  // record_token (sampler.odin:50-56)
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
}

}  // namespace

int sample_max_vocab() { return SAMPLE_MAX_VOCAB; }

hipError_t launch_sample(const float *logits, float *p, int n, SampleState *ss, int32_t *state, int32_t *tokens_out,
                         int32_t *pick, hipStream_t st) {
    if (n <= 0 || n > SAMPLE_MAX_VOCAB) return hipErrorInvalidValue;
    hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(SWG), 0, st, logits, p, n, ss, state, tokens_out, pick);
    return hipGetLastError();
}

}  // namespace oi
