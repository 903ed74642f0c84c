/*
 * oi_debug.h -- test hook of the HIP library: copies of the engine's
 * intermediate device buffers, for tests that check a stage of the token
 * step on its own.  No counterpart in the reference (its buffers are Odin
 * slices the tests can read directly).
 */
#ifndef OI_DEBUG_H
#define OI_DEBUG_H

#include <stdint.h>

#include "oi.h"

#ifdef __cplusplus
extern "C" {
#endif

enum {
    OI_BUF_XQ = 0,      /* quantized residual stream (token kernel) */
    OI_BUF_ATTQ = 1,    /* quantized attention output (token kernel) */
    OI_BUF_HBQ = 2,     /* quantized SwiGLU output (token kernel) */
    OI_BUF_SSQ = 3,     /* per-workgroup sums of squares (token kernel) */
    OI_BUF_Q = 4,       /* q, k, v projections of the last layer */
    OI_BUF_K = 5,
    OI_BUF_V = 6,
    OI_BUF_PART = 7,    /* attention partials [n_heads][chunks][head_dim + 4]: o, m, l, pad (token kernel;
                           the multi-kernel path uses a stride of head_dim + 2) */
    OI_BUF_LOGITS = 8,
    OI_BUF_STATE = 9,
    OI_BUF_AMVAL = 10,
    OI_BUF_AMIDX = 11,
    OI_BUF_TRACE = 12   /* token kernel stage trace (engine loaded with OI_STREAM_TRACE=1):
                           uint64 [1 + 6 n_layers + 1][workgroups][8], 100 MHz clock: 0 barrier
                           passed, 1 inputs loaded, 2 compute start, 4 compute done, 5 outputs
                           in LDS, 6 arrival (I/O wave or compute wave 0) */
};

/* Copy up to `bytes` of buffer `which` to host memory; returns the bytes
 * copied or a negative error code. */
int64_t oi_engine_debug_buffer(oi_engine *e, int32_t which, void *dst, int64_t bytes);

#ifdef __cplusplus
}
#endif
#endif /* OI_DEBUG_H */
