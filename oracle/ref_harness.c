/*
 * ref_harness.c — exports the reference engine's scalar CPU expert path.
 *
 * TEST INFRASTRUCTURE ONLY. oracle/Makefile compiles this file together
 * with the reference's own sources where they lie (csrc/core under the
 * reference tree, put on the include path by the Makefile) into
 * oracle/_ref/libwisp_ref.so. No reference source is copied: the engine
 * translation unit is #included from the reference tree at build time.
 *
 * It is built WITHOUT AVX-512 (-march=x86-64-v3) so the reference's
 * #else (scalar) branches are selected; its AVX-512 branches compute a
 * different function (16x gemv, skipped SwiGLU outputs).
 *
 * The wrappers call the reference's static functions:
 *   cpu_gemv_int4        csrc/core/wisp_engine.c:822-845
 *   cpu_gemv_f16         csrc/core/wisp_engine.c:630-645
 *   cpu_swiglu           csrc/core/wisp_engine.c:677-686
 *   cpu_gemv_t_f16       csrc/core/wisp_engine.c:647-658
 *   cpu_rmsnorm          csrc/core/wisp_engine.c:660-671
 *   cpu_residual_add     csrc/core/wisp_engine.c:673-675
 *   cpu_router_topk      csrc/core/wisp_engine.c:782-818
 *   cpu_expert_ffn       csrc/core/wisp_engine.c:1534-1561
 *   wisp_expert_fetch    csrc/core/wisp_engine.c:1138-1296 (tier policy)
 */
#include "wisp_engine.c"

void ref_gemv_int4(const uint8_t* packed, const uint16_t* scales,
                   const uint16_t* zeros, const float* x, float* y,
                   int rows, int cols, int gs) {
    cpu_gemv_int4(packed, scales, zeros, x, y, rows, cols, gs);
}

void ref_gemv_f16(const uint16_t* W, const float* x, float* y, int rows,
                  int cols) {
    cpu_gemv_f16((const wisp_half*)W, x, y, rows, cols);
}

void ref_swiglu(const float* g, const float* u, float* o, int n) {
    cpu_swiglu(g, u, o, n);
}

void ref_gemv_t_f16(const uint16_t* W, const float* x, float* y, int rows,
                    int cols) {
    cpu_gemv_t_f16((const wisp_half*)W, x, y, rows, cols);
}

void ref_rmsnorm(const float* x, const uint16_t* w, float* y, int n, float eps) {
    cpu_rmsnorm(x, (const wisp_half*)w, y, n, eps);
}

void ref_residual_add(float* x, const float* d, int n) {
    cpu_residual_add(x, d, n);
}

void ref_router_topk(const uint16_t* W, const uint16_t* bias, const float* x,
                     float* logits, int n_experts, int hidden, int top_k,
                     int* idx, float* w) {
    cpu_router_topk((const wisp_half*)W, (const wisp_half*)bias, x, logits,
                    n_experts, hidden, top_k, idx, w);
}

float ref_half_to_float(uint16_t h) { return wisp_half_to_float(h); }
uint16_t ref_float_to_half(float f) { return wisp_float_to_half(f); }

/* Parse a blob with the reference parser; fills 14 values:
 * rows[3], cols[3], packed_off[3], scales_off[3], group_size, total. */
int ref_parse_header(const void* blob, size_t size, uint64_t* out14) {
    WispErrCtx err;
    memset(&err, 0, sizeof(err));
    WispExpertMeta m;
    memset(&m, 0, sizeof(m));
    WispError e = wisp_expert_parse_header(blob, size, &m, &err);
    for (int i = 0; i < 3; i++) {
        out14[i] = m.rows[i];
        out14[3 + i] = m.cols[i];
        out14[6 + i] = m.packed_off[i];
        out14[9 + i] = m.scales_off[i];
    }
    out14[12] = m.group_size;
    out14[13] = m.total_bytes;
    return (int)e;
}

int ref_debug_probe(const char* path, int mat, int n, float* out) {
    WispErrCtx err;
    memset(&err, 0, sizeof(err));
    return (int)wisp_debug_expert_probe(path, mat, n, out, NULL, &err);
}

/* acc += w * expert(x), via the reference's cpu_expert_ffn on a minimal
 * engine that carries only what that function reads. */
int ref_expert_ffn(const void* blob, size_t size, const float* x, float* acc,
                   float w) {
    WispErrCtx err;
    memset(&err, 0, sizeof(err));
    WispExpertMeta meta;
    if (wisp_expert_parse_header(blob, size, &meta, &err) != WISP_OK)
        return (int)err.code;
    WispEngine* eng = (WispEngine*)calloc(1, sizeof(WispEngine));
    if (!eng) return (int)WISP_ERR_OOM;
    eng->expert_meta = &meta;
    size_t inter = meta.rows[0], hidden = meta.rows[2];
    eng->hs_gate = (float*)calloc(inter, sizeof(float));
    eng->hs_up = (float*)calloc(inter, sizeof(float));
    eng->hs_h = (float*)calloc(inter, sizeof(float));
    eng->hs_y = (float*)calloc(hidden, sizeof(float));
    int rc = (int)cpu_expert_ffn(eng, 0, (void*)blob, x, acc, w, &err);
    free(eng->hs_gate); free(eng->hs_up); free(eng->hs_h); free(eng->hs_y);
    free(eng);
    return rc;
}

int ref_selftest_lru(void) { return wisp_selftest_lru(); }

/* ---- tier policy trace --------------------------------------------------
 * A partial engine in GPU mode (experts_on_gpu = 1) whose "device" memory
 * is host memory (WISP_NO_CUDA shim), reading expert files from
 * <model_path>/experts/L###_E#####.bin exactly as the reference does. */
void* ref_tier_create(const char* model_path, int num_layers, int top_k,
                      size_t max_expert_bytes, size_t vram_budget,
                      size_t ram_budget) {
    WispEngine* eng = (WispEngine*)calloc(1, sizeof(WispEngine));
    WispErrCtx err;
    memset(&err, 0, sizeof(err));
    snprintf(eng->model_path, sizeof(eng->model_path), "%s", model_path);
    wisp_mutex_init(&eng->stats_mutex);
    eng->cfg.num_layers = num_layers;
    eng->cfg.top_k = top_k;
    eng->max_expert_bytes = max_expert_bytes;
    eng->experts_on_gpu = 1;
    eng->vram_cache = (LRUCache*)calloc(1, sizeof(LRUCache));
    eng->ram_cache = (LRUCache*)calloc(1, sizeof(LRUCache));
    eng->vram_budget = (VramBudget*)calloc(1, sizeof(VramBudget));
    lru_init(eng->vram_cache, vram_budget, TIER_VRAM, &err);
    lru_init(eng->ram_cache, ram_budget, TIER_RAM, &err);
    vram_budget_init(eng->vram_budget, vram_budget);
    eng->expert_meta = (WispExpertMeta*)calloc((size_t)num_layers,
                                               sizeof(WispExpertMeta));
    eng->scratch_slots = top_k + 2 > 16 ? 16 : top_k + 2;
    for (int i = 0; i < eng->scratch_slots; i++)
        eng->scratch_ring[i] = malloc(max_expert_bytes);
    return eng;
}

/* Returns the path taken: 0 VRAM hit, 1 RAM hit served by the scratch ring,
 * 2 RAM hit promoted into VRAM, 3 SSD miss placed in VRAM, 4 SSD miss
 * served by the scratch ring, -1 error. */
int ref_tier_fetch(void* h, uint32_t layer, uint32_t expert) {
    WispEngine* eng = (WispEngine*)h;
    WispErrCtx err;
    memset(&err, 0, sizeof(err));
    uint64_t v0 = eng->vram_hits, r0 = eng->ram_hits;
    void* p = wisp_expert_fetch(eng, layer, expert, &err);
    if (!p) return -1;
    int scratch = 0;
    for (int i = 0; i < eng->scratch_slots; i++)
        scratch |= (p == eng->scratch_ring[i]);
    if (eng->vram_hits != v0) return 0;
    if (eng->ram_hits != r0) return scratch ? 1 : 2;
    return scratch ? 4 : 3;
}

/* counts[0..4] = vram_hits, ram_hits, ssd_hits, vram entries, ram entries */
void ref_tier_stats(void* h, uint64_t* counts) {
    WispEngine* eng = (WispEngine*)h;
    counts[0] = eng->vram_hits;
    counts[1] = eng->ram_hits;
    counts[2] = eng->ssd_hits;
    counts[3] = eng->vram_cache->count;
    counts[4] = eng->ram_cache->count;
}
