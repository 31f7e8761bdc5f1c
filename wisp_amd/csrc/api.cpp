/*
 * api.cpp — host-only parts of the C-ABI: blob header parsing, the
 * profiling hook and the version string.
 */
#include <string.h>

#include "../../include/wisp_amd.h"

extern "C" {
hipEvent_t* wisp_amd__events = nullptr;
int wisp_amd__event_pairs = 0;
}

static uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
           ((uint32_t)p[3] << 24);
}
static uint64_t rd64(const uint8_t* p) { return (uint64_t)rd32(p) | ((uint64_t)rd32(p + 4) << 32); }

/* Header checks and section walk of csrc/core/wisp_engine.c:268-303:
 * magic 0x57455850, version 1, n_mats 3, then per matrix
 * {u32 rows, u32 cols, u64 packed, u64 scales, u64 zeros}; sections follow
 * the 120-byte header in order gate, up, down x [packed|scales|zeros]. */
extern "C" int wisp_expert_layout_from_blob(const void* host_blob, size_t blob_size,
                                            WispExpertLayout* out) {
    const uint8_t* b = (const uint8_t*)host_blob;
    if (!b || !out || blob_size < 120) return -1;
    if (rd32(b) != 0x57455850u || rd32(b + 4) != 1u || rd32(b + 20) != 3u) return -2;
    memset(out, 0, sizeof(*out));
    out->group_size = rd32(b + 16);
    uint64_t off = 120;
    for (int m = 0; m < 3; m++) {
        const uint8_t* mh = b + 24 + 32 * m;
        out->rows[m] = rd32(mh);
        out->cols[m] = rd32(mh + 4);
        out->packed_off[m] = off; off += rd64(mh + 8);
        out->scales_off[m] = off; off += rd64(mh + 16);
        out->zeros_off[m] = off;  off += rd64(mh + 24);
    }
    out->has_zeros = 1;
    out->total_bytes = off;
    return off > blob_size ? -3 : 0;
}

extern "C" void wisp_amd_set_kernel_events(hipEvent_t* events, int n_pairs) {
    wisp_amd__events = (events && n_pairs > 0) ? events : nullptr;
    wisp_amd__event_pairs = wisp_amd__events ? n_pairs : 0;
}

extern "C" const char* wisp_amd_version(void) { return "wisp_amd 0.1.0 (gfx950)"; }
