// stream_plan.h -- host planning of the persistent token kernel (stream_plan.cpp).
#pragma once
#include <string>
#include <vector>

#include "stream.h"

namespace oi {

struct PlanKind {
    SKind kind{};
    std::vector<SWave> waves;     // [G * S_NCW]
    std::vector<SWgRows> wgrows;  // [G]
    int max_wg_rows = 0;
};

// Plan one weight stage: `nseg` matrices of `types`/`rows` sharing row length
// K (GU: gate and up, planned as one segment of pairs).  own: rows owned per
// workgroup for WO / GU / DOWN.  False (and `why`) if the token kernel cannot
// run this stage.
bool plan_stream_kind(int kind, const int *types, int nseg, const int *rows, int K, int G, int own, PlanKind &pk,
                      std::string &why);

// One stage of the streams of compute waves [w0, w1): wave w's
// pk.waves[w].npieces KB at wdst[w - w0].  src[s] = GGUF blocks of segment s
// (GU: src[0] gate, src[1] up).
void repack_stream_kind(const PlanKind &pk, const uint8_t *const *src, int w0, int w1, uint8_t *const *wdst);

}  // namespace oi
