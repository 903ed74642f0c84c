// stream.h -- descriptors of the persistent token kernel (stream.hip), shared
// by the host planner (stream_plan.cpp) and the device code.
//
// One launch computes one token: embedding, every layer, logits and the
// greedy-argmax partials (reference: infer/forward.odin:17-146 and
// sampler/sampler.odin:79-89).  The grid is one workgroup per CU, all
// resident at once (cooperative launch).  A workgroup has S_NCW compute
// waves, S_NLD loader waves and one I/O wave:
//   * every compute wave has its share of every weight matrix of the token
//     laid out contiguously in consumption order (its stream); the loader
//     waves copy the streams into per-compute-wave LDS rings with 16-byte
//     register loads (many in flight) and publish fill counters in LDS, so
//     the compute waves read weights from LDS only and the loads run ahead
//     of the computation across stage barriers;
//   * compute waves issue no global memory traffic except the attention
//     K/V tile loads;
//   * the I/O wave does the coherent traffic: it loads each stage's input
//     vector (written by other workgroups in this launch) with device-scope
//     loads, stores the workgroup's outputs with device-scope stores, and
//     takes part in the grid barrier between stages (device-scope atomic
//     counters, no cache flushes).
// Weight loads run ahead of the computation by up to the ring size, across
// barriers, so HBM keeps streaming while a stage waits for its input.  (On
// gfx950, direct-to-LDS loads measured at most ~3.7 TB/s with 8 issuing
// waves per CU, 16-byte register loads ~7 TB/s: hence loader waves.)
#pragma once
#include <stdint.h>

#include "oi_kernels.h"

namespace oi {

constexpr int S_NCW = 8;                   // compute waves per workgroup
constexpr int S_NLD = 2;                   // loader waves per workgroup (fill the compute waves' rings)
constexpr int S_THREADS = 64 * (S_NCW + S_NLD + 1);  // + the I/O wave
constexpr int S_RING = 13;                 // ring pieces (1 KB) per compute wave
constexpr int S_RING_BYTES = S_RING * 1024;
constexpr int S_CP = 2;                    // pieces per loader request (chunk)
constexpr int S_NC = 32;                   // barrier counters (each in its own 256-byte line)
constexpr int S_MAXRUN = 4;                // row runs per compute wave per stage
constexpr int S_TR_SLOTS = 24;             // debugging trace words per (stage, workgroup)

// Stages that stream weights, in the order of a layer (+ the vocab projection).
enum StageKind : int32_t { SK_QKV = 0, SK_WO = 1, SK_GU = 2, SK_DOWN = 3, SK_VOCAB = 4, SK_N = 5 };

// Stream layout of one step: NR = 64/lpr rows x lpr units (64 weights each)
// of one block of a row, 64 lanes = one unit each.  Bytes per step:
//   Q4_K 2304: plane0 [64][16] (qs of the group pair, first 16 bytes),
//              plane1 [64][16], header [16][16] (d, dmin, 4 x 24-bit sc/m)
//   Q6_K 3360: planes ql-lo, ql-hi, qh [64][16] each, scales [16][16] (int8),
//              d [16][2] (f16)
//   Q8_0 4352: planes 0..3 [64][16] (int8 values 16c..16c+15), d [64][2][2]
// Lane l reads 16 bytes at l*16 of every plane and the header entry of its
// super-block at (l/4)*16, independent of lpr.  A SwiGLU pair step is the
// gate step followed by the up step.
constexpr int step_bytes(int type) { return type == T_Q4_K ? 2304 : type == T_Q6_K ? 3360 : 4352; }

struct SSeg {
    int32_t type;    // T_Q4_K, T_Q6_K or T_Q8_0
    int32_t rows;    // rows of the matrix
    int32_t vrow0;   // first virtual row of the segment in the stage
    int32_t pad;
};

struct SKind {
    int32_t nseg;
    int32_t K;       // row length
    int32_t lpr;     // lanes per row (power of two <= 64 dividing K/64)
    int32_t pair;    // 1: SwiGLU pairs (gate, up); a virtual row is one pair
    int64_t region;  // most bytes of one compute wave's stream in this stage (whole pieces)
    int64_t pad2;
    SSeg seg[3];
};

struct SRun {
    int32_t seg;
    int32_t row0;    // first row within the segment
    int32_t nrows;
    int32_t vrow;    // virtual row of row0 within the stage
};

// Work of one compute wave in one stage kind.
struct SWave {
    int32_t nruns;
    int32_t npieces;  // 1 KB pieces of the wave's stream in this stage
    int32_t pad[2];
    SRun run[S_MAXRUN];
};

// Virtual rows of a stage computed by one workgroup: [v0, v1).
struct SWgRows {
    int32_t v0, v1;
};

struct SLayer {
    int32_t plan[4];       // plan index (kinds / waves / wgrows) of each stage
    const float *attn_norm, *ffn_norm, *q_norm, *k_norm;
    uint16_t *kc, *vc;     // [n_kv_heads][seq_len][head_dim] f16
};

// Quantized activation vector (the inter-stage format), the LDS image the
// GEMV reads: per 16 elements (chunk C) a 16-bit integer q = 256 hi + lo per
// element (hi int8, lo 0..255) in two byte planes at chunk slot cslot(C), a
// float scale xs[C] (value = q * xs) and the float sum s16[C] of the values.
// 2.5 bytes per element.
constexpr int64_t qvec_bytes(int64_t K) { return K / 16 * 40; }

struct StreamArgs {
    const SLayer *layers;
    int32_t n_layers;
    int32_t G;                 // workgroups (= CUs)
    const uint8_t *wstream;    // weight streams: compute wave w's at wstream + w * wstride
    int64_t wstride;
    const int32_t *wpieces;    // [G * S_NCW] 1 KB pieces of each compute wave's stream
    int32_t vocab_plan;
    const float *output_norm;
    DMat emb;                  // token embedding (GEMV plane layout)
    const SKind *kinds;        // [plans]  (one plan per distinct stage kind + weight types)
    const SWave *waves;        // [plans][G * S_NCW]
    const SWgRows *wgrows;     // [plans][G]
    int32_t D, H, QD, KVD, HD, n_heads, n_kv, vocab, seq_len;
    int32_t rD, rH, rQ;        // rows owned per workgroup (multiples of 16) of x, hb, att
    float eps;
    const float2 *rope_cs;     // [seq_len][HD/2]
    float *q, *k, *v;          // raw projections of this token
    float *part;               // [n_heads][max_chunks][HD + 4] attention partials (o, m, l, pad)
    int32_t max_chunks;
    uint8_t *xq, *attq, *hbq;  // quantized vectors (qvec_bytes(D), (QD), (H))
    float *ssq;                // [G] partial sums of squares of the residual stream
    float *logits;             // [vocab]
    float *am_val;             // [G] argmax partials
    int32_t *am_idx;
    int32_t *state;            // ST_* words (oi_kernels.h) + the launch sequence
    int32_t *tokens;
    uint64_t *bar;             // [S_NC * 32] barrier counters
    int32_t finalize_only;     // reduce the pending argmax and stop
    int32_t yo_floats;         // most stage outputs of one workgroup
    uint64_t *trace;           // debugging (null: off): [stage][G][S_TR_SLOTS] clock stamps and counters
};

// state words used by the stream kernel beyond ST_*: launch sequence (64-bit
// at ST_SEQ), error flag
enum { ST_ERR = 6, ST_SEQ = 8, ST_SWORDS = 12 };
enum { S_ERR_TIMEOUT = 1 };

// host side (stream.hip)
hipError_t launch_stream(const StreamArgs &a, hipStream_t st);
size_t stream_lds_bytes(int kmax, int yo_floats);  // dynamic LDS of stream_kernel

}  // namespace oi
