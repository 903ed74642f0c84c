// stream_plan.cpp -- host planning for the persistent token kernel
// (stream.hip): which rows every compute wave computes in every weight stage,
// and the repack of the GGUF blocks into the compute waves' weight streams.
//
// Row assignment.  Stages whose output feeds the next GEMV through the
// producer-quantized vector (WO, GU, DOWN) give each workgroup the rows it
// owns (16-row chunks: rD / rH per workgroup) and split them evenly over its
// compute waves.  QKV and VOCAB, whose outputs are plain floats, split the
// concatenated rows of their matrices over all compute waves in proportion
// to bytes (Q6_K rows are 1.46x Q4_K rows), so every wave streams about the
// same amount.
//
// A compute wave's part of one stage in its stream: for each of its runs,
// for each step of NR = 64/lpr rows, for each block of lpr units of those
// rows, the step bytes of stream.h (SwiGLU pairs: gate step, then up step),
// padded to whole 1 KB pieces.  Rows past the end of a run inside a step are
// zero blocks.  The stream is the concatenation of these parts over the
// stages of a token (per layer QKV, WO, GU, DOWN, then VOCAB).
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "stream.h"
#include "stream_plan.h"

namespace oi {

static int pick_lpr(int K) {
    const int U = K / 64;
    int lpr = 64;
    while (lpr > 4 && U % lpr) lpr >>= 1;
    return U % lpr == 0 ? lpr : 0;
}

static double unit_bytes(int type) { return type == T_Q4_K ? 36.0 : type == T_Q6_K ? 52.5 : 68.0; }

// steps of one run and their bytes
static int64_t run_bytes(const SKind &k, const SRun &r) {
    const int NR = 64 / k.lpr, nb = (k.K / 64) / k.lpr;
    const int64_t steps = (int64_t)((r.nrows + NR - 1) / NR) * nb;
    return steps * step_bytes(k.seg[r.seg].type) * (k.pair ? 2 : 1);
}

static void finish_kind(PlanKind &pk) {
    int64_t maxp = 0;
    for (SWave &w : pk.waves) {
        int64_t b = 0;
        for (int i = 0; i < w.nruns; i++) b += run_bytes(pk.kind, w.run[i]);
        w.npieces = (int32_t)((b + 1023) / 1024);
        maxp = std::max<int64_t>(maxp, w.npieces);
    }
    pk.kind.region = maxp * 1024;
}

// push rows [v0, v1) of the stage's virtual rows as runs of wave w
static bool add_runs(PlanKind &pk, SWave &w, int v0, int v1) {
    for (int s = 0; s < pk.kind.nseg && v0 < v1; s++) {
        const SSeg &sg = pk.kind.seg[s];
        const int a = std::max(v0, sg.vrow0), b = std::min(v1, sg.vrow0 + sg.rows);
        if (a >= b) continue;
        if (w.nruns == S_MAXRUN) return false;
        SRun &r = w.run[w.nruns++];
        r.seg = s;
        r.row0 = a - sg.vrow0;
        r.nrows = b - a;
        r.vrow = a;
    }
    return true;
}

// byte-balanced split of all virtual rows over G * S_NCW waves
static bool plan_balanced(PlanKind &pk, int G) {
    const int NW = G * S_NCW;
    int nv = 0;
    for (int s = 0; s < pk.kind.nseg; s++) nv = std::max(nv, pk.kind.seg[s].vrow0 + pk.kind.seg[s].rows);
    std::vector<double> cum((size_t)nv + 1, 0.0);
    for (int s = 0; s < pk.kind.nseg; s++) {
        const SSeg &sg = pk.kind.seg[s];
        for (int r = 0; r < sg.rows; r++) cum[(size_t)sg.vrow0 + r + 1] = unit_bytes(sg.type) * (pk.kind.K / 64);
    }
    for (int v = 0; v < nv; v++) cum[(size_t)v + 1] += cum[(size_t)v];
    // whole steps of NR rows stay together (rows of a step share a wave)
    const int NR = 64 / pk.kind.lpr;
    std::vector<int> start((size_t)NW + 1, nv);
    int v = 0;
    for (int w = 0; w < NW; w++) {
        start[(size_t)w] = v;
        const double target = cum[(size_t)nv] * (w + 1) / NW;
        while (v < nv && cum[(size_t)std::min(nv, v + NR)] <= target + 1e-9) v = std::min(nv, v + NR);
        if (w == NW - 1) v = nv;
    }
    start[(size_t)NW] = nv;
    pk.waves.assign((size_t)NW, SWave{});
    pk.wgrows.assign((size_t)G, SWgRows{});
    for (int w = 0; w < NW; w++)
        if (!add_runs(pk, pk.waves[(size_t)w], start[(size_t)w], start[(size_t)w + 1])) return false;
    for (int g = 0; g < G; g++) pk.wgrows[(size_t)g] = {start[(size_t)g * S_NCW], start[(size_t)(g + 1) * S_NCW]};
    int maxrows = 0;
    for (int g = 0; g < G; g++) maxrows = std::max(maxrows, pk.wgrows[(size_t)g].v1 - pk.wgrows[(size_t)g].v0);
    pk.max_wg_rows = maxrows;
    return true;
}

// workgroup g computes rows [g*own, min(rows, (g+1)*own)), split evenly over its waves
static bool plan_owned(PlanKind &pk, int G, int own) {
    const int NW = G * S_NCW, rows = pk.kind.seg[0].rows, NR = 64 / pk.kind.lpr;
    pk.waves.assign((size_t)NW, SWave{});
    pk.wgrows.assign((size_t)G, SWgRows{});
    pk.max_wg_rows = 0;
    for (int g = 0; g < G; g++) {
        const int r0 = std::min(rows, g * own), r1 = std::min(rows, (g + 1) * own);
        pk.wgrows[(size_t)g] = {r0, r1};
        pk.max_wg_rows = std::max(pk.max_wg_rows, r1 - r0);
        const int steps = (r1 - r0 + NR - 1) / NR;
        for (int w = 0; w < S_NCW; w++) {
            const int s0 = steps * w / S_NCW, s1 = steps * (w + 1) / S_NCW;
            const int a = std::min(r1, r0 + s0 * NR), b = std::min(r1, r0 + s1 * NR);
            if (a < b && !add_runs(pk, pk.waves[(size_t)g * S_NCW + w], a, b)) return false;
        }
    }
    return true;
}

static bool type_ok(int t) { return t == T_Q4_K || t == T_Q6_K || t == T_Q8_0; }

bool plan_stream_kind(int kind, const int *types, int nseg, const int *rows, int K, int G, int own, PlanKind &pk,
                      std::string &why) {
    pk = PlanKind{};
    SKind &k = pk.kind;
    k.K = K;
    k.lpr = pick_lpr(K);
    if (K % 256 || k.lpr == 0) {
        why = "row length " + std::to_string(K) + " not supported by the token kernel";
        return false;
    }
    k.pair = kind == SK_GU;
    k.nseg = k.pair ? 1 : nseg;
    int vrow = 0;
    for (int s = 0; s < k.nseg; s++) {
        if (!type_ok(types[s])) {
            why = "weight type not supported by the token kernel";
            return false;
        }
        // a compute wave holds one step in its ring while the loader needs
        // room for a whole chunk beyond it
        const int sb = step_bytes(types[s]) * (k.pair ? 2 : 1);
        if ((sb + 1023) / 1024 + S_CP > S_RING) {
            why = "weight step larger than the token kernel's ring";
            return false;
        }
        k.seg[s].type = types[s];
        k.seg[s].rows = rows[s];
        k.seg[s].vrow0 = vrow;
        vrow += rows[s];
    }
    if (k.pair && types[0] != types[1]) {
        why = "gate and up weights of different types";
        return false;
    }
    const bool ok = (kind == SK_QKV || kind == SK_VOCAB) ? plan_balanced(pk, G) : plan_owned(pk, G, own);
    if (!ok) {
        why = "row plan needs more runs per wave than supported";
        return false;
    }
    finish_kind(pk);
    return true;
}

// ------------------------------------------------------------- repack --
// Device form of a Q4_K header (see DMat in oi_kernels.h).
void q4k_header(const uint8_t *blk, uint8_t *out);

static size_t block_bytes(int type) { return type == T_Q4_K ? 144 : type == T_Q6_K ? 210 : 34; }

// one step (NR rows x lpr units, block b) of matrix `src` (GGUF blocks,
// row length K) at rows r0.. (rows >= nrows are zero), into out
static void write_step(int type, const uint8_t *src, int K, int lpr, int r0, int nrows, int b, uint8_t *out) {
    const int NR = 64 / lpr;
    const size_t row_bytes = (size_t)K / (type == T_Q8_0 ? 32 : 256) * block_bytes(type);
    std::memset(out, 0, (size_t)step_bytes(type));
    for (int lane = 0; lane < 64; lane++) {
        const int i = lane / lpr, j = lane % lpr;
        if (i >= nrows) continue;
        const uint8_t *row = src + (size_t)(r0 + i) * row_bytes;
        const int u = b * lpr + j;
        if (type == T_Q4_K) {
            const uint8_t *blk = row + (size_t)(u >> 2) * 144;
            const int p = u & 3;
            std::memcpy(out + 16 * lane, blk + 16 + 32 * p, 16);
            std::memcpy(out + 1024 + 16 * lane, blk + 32 + 32 * p, 16);
            if ((lane & 3) == 0) q4k_header(blk, out + 2048 + 16 * (lane >> 2));
        } else if (type == T_Q6_K) {
            const uint8_t *blk = row + (size_t)(u >> 2) * 210;  // ql[128] qh[64] sc[16] d
            const int h = (u >> 1) & 1, l0 = 16 * (u & 1);
            std::memcpy(out + 16 * lane, blk + 64 * h + l0, 16);
            std::memcpy(out + 1024 + 16 * lane, blk + 64 * h + 32 + l0, 16);
            std::memcpy(out + 2048 + 16 * lane, blk + 128 + 32 * h + l0, 16);
            if ((lane & 3) == 0) {
                std::memcpy(out + 3072 + 16 * (lane >> 2), blk + 192, 16);
                std::memcpy(out + 3328 + 2 * (lane >> 2), blk + 208, 2);
            }
        } else {  // Q8_0: unit u = blocks 2u, 2u+1
            for (int c = 0; c < 4; c++) {
                const uint8_t *blk = row + (size_t)(2 * u + (c >> 1)) * 34;
                std::memcpy(out + 1024 * c + 16 * lane, blk + 2 + 16 * (c & 1), 16);
            }
            std::memcpy(out + 4096 + 4 * lane, row + (size_t)(2 * u) * 34, 2);
            std::memcpy(out + 4096 + 4 * lane + 2, row + (size_t)(2 * u + 1) * 34, 2);
        }
    }
}

void repack_stream_kind(const PlanKind &pk, const uint8_t *const *src, int w0, int w1, uint8_t *const *wdst) {
    const SKind &k = pk.kind;
    const int NR = 64 / k.lpr, nb = (k.K / 64) / k.lpr;
    for (int w = w0; w < w1; w++) {
        const SWave &wv = pk.waves[(size_t)w];
        uint8_t *out = wdst[w - w0];
        std::memset(out, 0, (size_t)wv.npieces * 1024);
        for (int i = 0; i < wv.nruns; i++) {
            const SRun &r = wv.run[i];
            const int type = k.seg[r.seg].type, sb = step_bytes(type);
            for (int rs = 0; rs < (r.nrows + NR - 1) / NR; rs++) {
                const int row0 = r.row0 + rs * NR, n = std::min(NR, r.nrows - rs * NR);
                for (int b = 0; b < nb; b++) {
                    if (k.pair) {
                        write_step(type, src[0], k.K, k.lpr, row0, n, b, out);
                        write_step(type, src[1], k.K, k.lpr, row0, n, b, out + sb);
                        out += 2 * sb;
                    } else {
                        write_step(type, src[r.seg], k.K, k.lpr, row0, n, b, out);
                        out += sb;
                    }
                }
            }
        }
    }
}

}  // namespace oi
