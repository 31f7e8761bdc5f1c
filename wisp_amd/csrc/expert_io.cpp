/*
 * expert_io.cpp — real-weight ingestion on the host (C++): the converter's
 * group-wise int4 quantizer, the expert blob writer, and the expert file
 * reader and writer.
 *
 * wisp_quantize_int4 restates quantize_int4 (wisp/converter/quantizer.py:
 * 46-86) in fp32 scalar arithmetic that gives the same bytes as the
 * reference's torch ops: per group of group_size consecutive elements of
 * the row-major matrix (the last group padded with the last element),
 *     zero  = (max + min) / 2               fp32
 *     scale = max((max - min) / 15, 1e-8)   fp32
 *     q     = clamp(round_half_even((x - zero) / scale) + 8, 0, 15)
 * with scale and zero stored as fp16 (round to nearest even) and q packed
 * two per byte, low nibble first. q uses the fp32 scale and zero, not the
 * stored fp16 ones, as the reference does.
 *
 * The blob layout is the reference's expert file (wisp/converter/
 * partitioner.py:11-27, 56-89; parsed by csrc/core/wisp_engine.c:268-303):
 * a 24-byte header {magic 0x57455850, version 1, layer, expert, group
 * size, n_mats 3}, three 32-byte matrix headers {rows, cols, packed bytes,
 * scale bytes, zero bytes}, then [packed][scales][zeros] for gate, up and
 * down. Files are <model>/experts/L%03u_E%05u.bin, read whole as
 * read_expert_ssd does (csrc/core/wisp_engine.c:351-380).
 */
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

#include "../../include/wisp_amd.h"

namespace {

float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0x1F) {
        bits = sign | 0x7F800000u | (m << 13);
    } else if (e != 0) {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    } else {
        /* zero or subnormal: m * 2^-24 is exact in fp32 */
        float v = (float)m * (1.0f / 16777216.0f);
        memcpy(&bits, &v, 4);
        bits |= sign;
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* fp32 -> fp16, round to nearest even, overflow to inf (what a tensor cast
 * to float16 does). */
uint16_t float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t a = x & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return sign | 0x7E00u;            /* NaN */
    if (a >= 0x47800000u) return sign | 0x7C00u;           /* >= 2^16 (and inf) */
    if (a >= 0x38800000u) {                                /* fp16 normal range */
        const uint32_t exp = (a >> 23) - 112u;             /* rebias 127 -> 15 */
        uint32_t h = (exp << 10) | ((a & 0x7FFFFFu) >> 13);
        const uint32_t rem = a & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;   /* may carry into inf */
        return sign | (uint16_t)h;
    }
    /* subnormal or zero: |f| * 2^24 is exact, then round to an integer */
    float v;
    memcpy(&v, &a, 4);
    return sign | (uint16_t)nearbyintf(v * 16777216.0f);
}

float load_w(const void* w, int dtype, size_t i) {
    if (dtype == WISP_WEIGHT_F32) return ((const float*)w)[i];
    const uint16_t b = ((const uint16_t*)w)[i];
    if (dtype == WISP_WEIGHT_F16) return half_to_float(b);
    const uint32_t bits = (uint32_t)b << 16;                /* bf16 */
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Groups [g0, g1) of the flat matrix. Returns false on a non-finite value. */
bool quantize_groups(const void* w, int dtype, size_t n, uint32_t gs, size_t g0, size_t g1,
                     uint8_t* q, uint16_t* scales, uint16_t* zeros) {
    for (size_t g = g0; g < g1; g++) {
        const size_t a = g * gs, b = std::min(n, a + gs);
        float mx = load_w(w, dtype, a), mn = mx;
        for (size_t i = a; i < b; i++) {
            const float v = load_w(w, dtype, i);
            if (!isfinite(v)) return false;
            mx = v > mx ? v : mx;
            mn = v < mn ? v : mn;
        }
        const float zero = (mx + mn) / 2.0f;
        float scale = (mx - mn) / 15.0f;
        if (scale < 1e-8f) scale = 1e-8f;
        for (size_t i = a; i < b; i++) {
            const float d = load_w(w, dtype, i) - zero;
            float t = nearbyintf(d / scale) + 8.0f;   /* round half to even */
            t = t < 0.0f ? 0.0f : (t > 15.0f ? 15.0f : t);
            q[i] = (uint8_t)t;
        }
        scales[g] = float_to_half(scale);
        zeros[g] = float_to_half(zero);
    }
    return true;
}

void wr32(uint8_t* p, uint32_t v) { memcpy(p, &v, 4); }
void wr64(uint8_t* p, uint64_t v) { memcpy(p, &v, 8); }

}  // namespace

extern "C" int wisp_quantize_int4(const void* w, int dtype, uint32_t rows, uint32_t cols,
                                  uint32_t group_size, uint8_t* packed, wisp_half* scales,
                                  wisp_half* zeros) {
    if (!w || !packed || !scales || !zeros || rows == 0 || cols == 0 || group_size == 0 ||
        (dtype != WISP_WEIGHT_F32 && dtype != WISP_WEIGHT_F16 && dtype != WISP_WEIGHT_BF16))
        return -1;
    const size_t n = (size_t)rows * cols;
    const size_t n_groups = (n + group_size - 1) / group_size;
    std::vector<uint8_t> q(n);
    /* groups are independent: split them over threads for large matrices */
    unsigned nt = n >= ((size_t)1 << 20) ? std::thread::hardware_concurrency() : 1;
    nt = std::max(1u, std::min(nt, 32u));
    std::vector<char> ok(nt, 1);
    std::vector<std::thread> pool;
    const size_t per = (n_groups + nt - 1) / nt;
    for (unsigned t = 0; t < nt; t++) {
        const size_t g0 = std::min(n_groups, t * per), g1 = std::min(n_groups, g0 + per);
        auto job = [&, t, g0, g1]() {
            ok[t] = quantize_groups(w, dtype, n, group_size, g0, g1, q.data(), scales, zeros);
        };
        if (t + 1 == nt) job();
        else pool.emplace_back(job);
    }
    for (auto& th : pool) th.join();
    for (char o : ok)
        if (!o) return -2;
    for (size_t i = 0; i + 1 < n; i += 2) packed[i / 2] = (uint8_t)(q[i] | (q[i + 1] << 4));
    if (n % 2) packed[n / 2] = q[n - 1];   /* odd count: high nibble 0 */
    return 0;
}

extern "C" size_t wisp_expert_blob_bytes(const uint32_t rows[3], const uint32_t cols[3],
                                         uint32_t group_size) {
    if (!rows || !cols || group_size == 0) return 0;
    size_t total = 120;
    for (int m = 0; m < 3; m++) {
        const size_t n = (size_t)rows[m] * cols[m];
        const size_t ng = (n + group_size - 1) / group_size;
        total += (n + 1) / 2 + 4 * ng;
    }
    return total;
}

extern "C" size_t wisp_expert_blob_write(void* dst, size_t capacity, uint32_t layer,
                                         uint32_t expert, uint32_t group_size,
                                         const uint32_t rows[3], const uint32_t cols[3],
                                         const uint8_t* const packed[3],
                                         const wisp_half* const scales[3],
                                         const wisp_half* const zeros[3]) {
    const size_t total = wisp_expert_blob_bytes(rows, cols, group_size);
    if (!dst || total == 0 || capacity < total || !packed || !scales || !zeros) return 0;
    uint8_t* b = (uint8_t*)dst;
    wr32(b, 0x57455850u);
    wr32(b + 4, 1u);
    wr32(b + 8, layer);
    wr32(b + 12, expert);
    wr32(b + 16, group_size);
    wr32(b + 20, 3u);
    size_t off = 120;
    for (int m = 0; m < 3; m++) {
        const size_t n = (size_t)rows[m] * cols[m];
        const size_t ng = (n + group_size - 1) / group_size;
        const size_t pb = (n + 1) / 2, sb = 2 * ng;
        uint8_t* mh = b + 24 + 32 * m;
        wr32(mh, rows[m]);
        wr32(mh + 4, cols[m]);
        wr64(mh + 8, pb);
        wr64(mh + 16, sb);
        wr64(mh + 24, sb);
        memcpy(b + off, packed[m], pb);
        memcpy(b + off + pb, scales[m], sb);
        memcpy(b + off + pb + sb, zeros[m], sb);
        off += pb + 2 * sb;
    }
    return off;
}

extern "C" size_t wisp_expert_quantize_blob(const void* gate, const void* up, const void* down,
                                            int dtype, uint32_t inter, uint32_t hidden,
                                            uint32_t group_size, uint32_t layer, uint32_t expert,
                                            void* dst, size_t capacity) {
    const uint32_t rows[3] = {inter, inter, hidden}, cols[3] = {hidden, hidden, inter};
    const size_t total = wisp_expert_blob_bytes(rows, cols, group_size);
    if (!gate || !up || !down || !dst || total == 0 || capacity < total) return 0;
    const void* src[3] = {gate, up, down};
    const uint8_t* pk[3];
    const wisp_half* sc[3];
    const wisp_half* zr[3];
    std::vector<std::vector<uint8_t>> tmp(3);
    for (int m = 0; m < 3; m++) {
        const size_t n = (size_t)rows[m] * cols[m];
        const size_t ng = (n + group_size - 1) / group_size;
        tmp[m].resize((n + 1) / 2 + 4 * ng);
        uint8_t* p = tmp[m].data();
        if (wisp_quantize_int4(src[m], dtype, rows[m], cols[m], group_size, p,
                               (wisp_half*)(p + (n + 1) / 2),
                               (wisp_half*)(p + (n + 1) / 2 + 2 * ng)) != 0)
            return 0;
        pk[m] = p;
        sc[m] = (const wisp_half*)(p + (n + 1) / 2);
        zr[m] = (const wisp_half*)(p + (n + 1) / 2 + 2 * ng);
    }
    return wisp_expert_blob_write(dst, capacity, layer, expert, group_size, rows, cols, pk, sc,
                                  zr);
}

extern "C" int wisp_expert_file_path(char* out, size_t capacity, const char* model_path,
                                     uint32_t layer, uint32_t expert) {
    if (!out || !model_path || capacity == 0) return -1;
    const int k = snprintf(out, capacity, "%s/experts/L%03u_E%05u.bin", model_path, layer, expert);
    return (k < 0 || (size_t)k >= capacity) ? -1 : 0;
}

extern "C" int64_t wisp_expert_file_read(const char* model_path, uint32_t layer, uint32_t expert,
                                         void* dst, size_t max_bytes) {
    char path[1200];
    if (!dst || wisp_expert_file_path(path, sizeof(path), model_path, layer, expert) != 0)
        return WISP_IO_BAD_ARGUMENT;
    FILE* f = fopen(path, "rb");
    if (!f) return WISP_IO_MISSING;
    long size = -1;
    if (fseek(f, 0, SEEK_END) == 0) size = ftell(f);
    if (size <= 0 || (size_t)size > max_bytes || fseek(f, 0, SEEK_SET) != 0) {
        fclose(f);
        return WISP_IO_TOO_LARGE;
    }
    const size_t got = fread(dst, 1, (size_t)size, f);
    fclose(f);
    if (got != (size_t)size) return WISP_IO_SHORT_READ;
    return (int64_t)got;
}

extern "C" int wisp_expert_file_write(const char* model_path, uint32_t layer, uint32_t expert,
                                      const void* blob, size_t bytes) {
    char path[1200], tmp[1210];
    if (!blob || bytes == 0 ||
        wisp_expert_file_path(path, sizeof(path), model_path, layer, expert) != 0)
        return WISP_IO_BAD_ARGUMENT;
    snprintf(tmp, sizeof(tmp), "%s.tmp", path);
    FILE* f = fopen(tmp, "wb");
    if (!f) return WISP_IO_MISSING;
    const size_t put = fwrite(blob, 1, bytes, f);
    const int closed = fclose(f);
    if (put != bytes || closed != 0 || rename(tmp, path) != 0) {
        remove(tmp);
        return WISP_IO_SHORT_READ;
    }
    return 0;
}
