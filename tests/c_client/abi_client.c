/*
 * abi_client.c -- a plain C11 caller of libadambridge_hip.so (test program).
 *
 * It uses the library the way the reference's own binding uses its native
 * kernel library (adambridge/native.py:273-435, engine.py:862-884): it fills
 * adambridge_group / adambridge_segment structs from include/adambridge_hip.h,
 * creates a pool, calls adambridge_multi_step once per step for all segments
 * together and synchronises.  No Python and no torch: device buffers come
 * from hipMalloc, and the header is compiled as C.
 *
 *   abi_client abi                 no GPU: version, struct sizes, SIMD-level
 *                                  switch, argument checks (nothing reaches a device)
 *   abi_client gpu ORACLE.so       three segments (AdamW BF16 moments; AdamW FP8 moments
 *                                  with an FP24 master at a non-zero offset; Lion), three
 *                                  multi_step steps, one multi_apply with explicit
 *                                  coefficients, then one fused_adamw on the first tensor;
 *                                  after each, every buffer compared byte for byte with the
 *                                  same update computed by the CPU oracle (oracle/liboracle.so,
 *                                  the checker: abo_multi_step / abo_multi_apply on host copies)
 *
 * Exit status 0 when every check passes; the failing check is printed.
 */
#include <dlfcn.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "adambridge_hip.h"

_Static_assert(sizeof(adambridge_hparams) == 40, "hparams: kernels.c:77-88");
_Static_assert(sizeof(adambridge_group) == 56, "group: kernels.c:736-745");
_Static_assert(sizeof(adambridge_segment) == 128, "segment: kernels.c:747-769");

static int failures = 0;

#define CHECK(cond, ...)                                   \
    do {                                                   \
        if (!(cond)) {                                     \
            fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            fprintf(stderr, __VA_ARGS__);                  \
            fputc('\n', stderr);                           \
            ++failures;                                    \
        }                                                  \
    } while (0)

/* ------------------------------------------------------------------ no GPU */

static int run_abi(void)
{
    CHECK(adambridge_abi_version() == ADAMBRIDGE_ABI_VERSION, "abi_version %d", adambridge_abi_version());
    CHECK(adambridge_hparams_size() == (int)sizeof(adambridge_hparams), "hparams_size");
    CHECK(adambridge_group_size() == (int)sizeof(adambridge_group), "group_size");
    CHECK(adambridge_segment_size() == (int)sizeof(adambridge_segment), "segment_size");
    CHECK(adambridge_backend() != NULL && adambridge_backend()[0] != '\0', "backend");

    const int level = adambridge_simd_level();
    CHECK(adambridge_set_simd_level(0) == 0 && adambridge_simd_level() == 0, "set_simd_level(0)");
    CHECK(adambridge_set_simd_level(1) == 1, "set_simd_level(1)");
    CHECK(adambridge_set_simd_level(level) == level, "restore simd level");

    /* kernels.c:1537-1553: every segment is checked before anything is enqueued, so these
     * return without touching a device (the pointers are never dereferenced) */
    static char dummy[256];
    adambridge_group grp = {1e-3, 0.9, 0.999, 1e-8, 0.01, 0, 0, 0};
    adambridge_segment s;
    memset(&s, 0, sizeof s);
    s.p = dummy; s.g = dummy; s.m = dummy; s.v = dummy; s.group = &grp;
    s.n = 16; s.step = 1;
    s.g_dtype = ADAMBRIDGE_DT_BF16; s.mv_dtype = ADAMBRIDGE_DT_BF16;
    s.out_dtype = ADAMBRIDGE_DT_NONE; s.algorithm = ADAMBRIDGE_ALGO_ADAMW; s.p_dtype = ADAMBRIDGE_DT_F32;
    adambridge_segment* one[1] = {&s};
    struct { const char* what; int field; int value; int code; } cases[] = {
        {"negative n", 0, -1, ADAMBRIDGE_EBADN},
        {"unknown algorithm", 1, 7, ADAMBRIDGE_EALGO},
        {"unknown p_dtype", 2, 17, ADAMBRIDGE_EPDTYPE},
        {"NULL gradient", 3, 0, ADAMBRIDGE_ENULL},
        {"gradient dtype FP8", 4, ADAMBRIDGE_DT_FP8, ADAMBRIDGE_EGDTYPE},
        {"moment dtype F24", 5, ADAMBRIDGE_DT_F24, ADAMBRIDGE_EMVDTYPE},
        {"out dtype FP8", 6, ADAMBRIDGE_DT_FP8, ADAMBRIDGE_EOUTDTYPE},
        {"out dtype BF16 without out", 6, ADAMBRIDGE_DT_BF16, ADAMBRIDGE_EOUTNULL},
        {"FP8 moments without scales", 5, ADAMBRIDGE_DT_FP8, ADAMBRIDGE_ESCALES},
        {"no group", 7, 0, ADAMBRIDGE_EGROUP},
        {"negative offset", 8, -128, ADAMBRIDGE_EOFFSET},
    };
    for (size_t k = 0; k < sizeof cases / sizeof cases[0]; ++k) {
        adambridge_segment b = s;
        switch (cases[k].field) {
            case 0: b.n = cases[k].value; break;
            case 1: b.algorithm = cases[k].value; break;
            case 2: b.p_dtype = cases[k].value; break;
            case 3: b.g = NULL; break;
            case 4: b.g_dtype = cases[k].value; break;
            case 5: b.mv_dtype = cases[k].value; break;
            case 6: b.out_dtype = cases[k].value; break;
            case 7: b.group = NULL; break;
            case 8: b.offset = cases[k].value; break;
        }
        adambridge_segment* bad[2] = {&s, &b};   /* a valid segment first: nothing may run */
        const int rc = adambridge_multi_step(NULL, bad, 2, 0);
        CHECK(rc == cases[k].code, "%s: code %d, expected %d", cases[k].what, rc, cases[k].code);
    }
    CHECK(adambridge_multi_step(NULL, NULL, 1, 0) == ADAMBRIDGE_EBADN, "NULL segment array");
    CHECK(adambridge_multi_step(NULL, one, 0, 0) == 0, "zero segments");
    CHECK(adambridge_multi_apply(NULL, one, NULL, 1, 0) == ADAMBRIDGE_EBADN, "multi_apply without hparams");
    return failures;
}

/* ---------------------------------------------------------------- with GPU */

typedef int (*oracle_multi_step_fn)(adambridge_segment* const*, int32_t, int64_t, int32_t);
typedef int (*oracle_multi_apply_fn)(adambridge_segment* const*, const adambridge_hparams*, int32_t, int64_t,
                                     int32_t);

static uint64_t rng_state = 0x243F6A8885A308D3ull;

static uint64_t next64(void)   /* splitmix64 */
{
    uint64_t z = (rng_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static float uniform(float lo, float hi)
{
    return lo + (hi - lo) * (float)((next64() >> 40) * 0x1p-24);
}

static uint32_t bits_of(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }

/* A buffer held twice: host (updated by the oracle) and device (updated by the library). */
typedef struct { void* host; void* dev; size_t bytes; const char* name; } Buf;

#define MAX_BUFS 32
static Buf bufs[MAX_BUFS];
static int nbufs = 0;

static Buf* new_buf(size_t bytes, const char* name)
{
    if (nbufs == MAX_BUFS) { fprintf(stderr, "too many buffers\n"); exit(2); }
    Buf* b = &bufs[nbufs++];
    b->host = calloc(bytes ? bytes : 1, 1);
    b->bytes = bytes;
    b->name = name;
    if (!b->host || hipMalloc(&b->dev, bytes ? bytes : 1) != hipSuccess) {
        fprintf(stderr, "allocation of %s (%zu bytes) failed\n", name, bytes);
        exit(2);
    }
    return b;
}

static int upload(const Buf* b)
{
    return hipMemcpy(b->dev, b->host, b->bytes, hipMemcpyHostToDevice) == hipSuccess ? 0 : -1;
}

/* Device bytes equal to the host bytes; reports the first differing byte. */
static int compare(const Buf* b, int step)
{
    unsigned char* got = (unsigned char*)malloc(b->bytes ? b->bytes : 1);
    if (!got || hipMemcpy(got, b->dev, b->bytes, hipMemcpyDeviceToHost) != hipSuccess) {
        fprintf(stderr, "read-back of %s failed\n", b->name);
        exit(2);
    }
    const unsigned char* want = (const unsigned char*)b->host;
    size_t first = b->bytes, count = 0;
    for (size_t i = 0; i < b->bytes; ++i) {
        if (got[i] != want[i]) {
            if (first == b->bytes) first = i;
            ++count;
        }
    }
    free(got);
    CHECK(count == 0, "step %d, %s: %zu of %zu bytes differ, first at byte %zu", step, b->name, count, b->bytes,
          first);
    return count == 0;
}

/* One segment over host and device buffers. */
typedef struct {
    adambridge_segment host, dev;
    Buf *p, *p_lo, *g, *m, *v, *ms, *vs, *out;
} Seg;

static void attach(Seg* s)
{
#define PTRS(field, buf) s->host.field = (buf) ? (buf)->host : NULL; s->dev.field = (buf) ? (buf)->dev : NULL
    PTRS(p, s->p);
    PTRS(p_lo, s->p_lo);
    PTRS(g, s->g);
    PTRS(m, s->m);
    PTRS(v, s->v);
    PTRS(m_scale, s->ms);
    PTRS(v_scale, s->vs);
    PTRS(out, s->out);
#undef PTRS
}

static void fill_gradient(Seg* s, float zero_fraction)
{
    const int64_t n = s->host.n;
    for (int64_t i = 0; i < n; ++i) {
        const float x = uniform(0.0f, 1.0f) < zero_fraction ? 0.0f : uniform(-2.0f, 2.0f) * 1e-2f;
        if (s->host.g_dtype == ADAMBRIDGE_DT_BF16) ((uint16_t*)s->g->host)[i] = (uint16_t)(bits_of(x) >> 16);
        else ((float*)s->g->host)[i] = x;
    }
}

static int run_gpu(const char* oracle_path)
{
    void* lib = dlopen(oracle_path, RTLD_NOW | RTLD_LOCAL);
    if (!lib) { fprintf(stderr, "dlopen %s: %s\n", oracle_path, dlerror()); return 2; }
    oracle_multi_step_fn oracle_step = (oracle_multi_step_fn)(uintptr_t)dlsym(lib, "abo_multi_step");
    oracle_multi_apply_fn oracle_apply = (oracle_multi_apply_fn)(uintptr_t)dlsym(lib, "abo_multi_apply");
    int (*oracle_segment_size)(void) = (int (*)(void))(uintptr_t)dlsym(lib, "abo_segment_size");
    if (!oracle_step || !oracle_apply || !oracle_segment_size ||
        oracle_segment_size() != (int)sizeof(adambridge_segment)) {
        fprintf(stderr, "oracle library does not match the segment layout\n");
        return 2;
    }
    if (hipSetDevice(0) != hipSuccess) { fprintf(stderr, "hipSetDevice(0) failed\n"); return 2; }

    const int level = adambridge_simd_level();
    const int64_t width = level == 2 ? 16 : level == 1 ? 8 : 0;
    adambridge_group adamw_rne = {1e-3, 0.9, 0.999, 1e-8, 0.01, 42, 0, 0};
    adambridge_group adamw_sr = {3e-4, 0.8, 0.95, 1e-6, 0.1, 7, 1, 0};
    adambridge_group lion = {1e-4, 0.9, 0.99, 0.0, 0.05, 9, 1, 0};

    Seg segs[3];
    memset(segs, 0, sizeof segs);

    /* 0: AdamW, FP32 master, BF16 moments (nearest), BF16 gradient and output;
     *    n leaves a scalar tail after the 16-wide fused range */
    {
        Seg* s = &segs[0];
        const int64_t n = 1000003;
        s->host.n = n; s->host.index = 0; s->host.offset = 0; s->host.group = &adamw_rne;
        s->host.g_dtype = ADAMBRIDGE_DT_BF16; s->host.mv_dtype = ADAMBRIDGE_DT_BF16;
        s->host.out_dtype = ADAMBRIDGE_DT_BF16; s->host.algorithm = ADAMBRIDGE_ALGO_ADAMW;
        s->host.p_dtype = ADAMBRIDGE_DT_F32;
        s->p = new_buf((size_t)n * 4, "seg0 master");
        s->g = new_buf((size_t)n * 2, "seg0 gradient");
        s->m = new_buf((size_t)n * 2, "seg0 m");
        s->v = new_buf((size_t)n * 2, "seg0 v");
        s->out = new_buf((size_t)n * 2, "seg0 out");
        for (int64_t i = 0; i < n; ++i) ((float*)s->p->host)[i] = uniform(-1.0f, 1.0f);
    }
    /* 1: AdamW, FP24 master, FP8 moments (stochastic rounding of both), FP32 gradient, BF16
     *    output; a chunk at
     *    element offset 384 of its parameter, ragged last block */
    {
        Seg* s = &segs[1];
        const int64_t n = 300001, blocks = (n + 127) / 128;
        s->host.n = n; s->host.index = 1; s->host.offset = 384; s->host.group = &adamw_sr;
        s->host.g_dtype = ADAMBRIDGE_DT_F32; s->host.mv_dtype = ADAMBRIDGE_DT_FP8;
        s->host.out_dtype = ADAMBRIDGE_DT_BF16; s->host.algorithm = ADAMBRIDGE_ALGO_ADAMW;
        s->host.p_dtype = ADAMBRIDGE_DT_F24;
        s->p = new_buf((size_t)n * 2, "seg1 master hi");
        s->p_lo = new_buf((size_t)n, "seg1 master lo");
        s->g = new_buf((size_t)n * 4, "seg1 gradient");
        s->m = new_buf((size_t)blocks * 128, "seg1 m codes");
        s->v = new_buf((size_t)blocks * 128, "seg1 v codes");
        s->ms = new_buf((size_t)blocks * 4, "seg1 m scales");
        s->vs = new_buf((size_t)blocks * 4, "seg1 v scales");
        s->out = new_buf((size_t)n * 2, "seg1 out");
        for (int64_t i = 0; i < n; ++i) {
            const uint32_t b = bits_of(uniform(-1.0f, 1.0f));
            ((uint16_t*)s->p->host)[i] = (uint16_t)(b >> 16);
            ((uint8_t*)s->p_lo->host)[i] = (uint8_t)(b >> 8);
        }
        for (int64_t k = 0; k < blocks; ++k) ((float*)s->ms->host)[k] = ((float*)s->vs->host)[k] = 1.0f;
    }
    /* 2: Lion, FP32 master, BF16 moment (stochastic rounding), BF16 gradient with exact zeros,
     *    no output copy */
    {
        Seg* s = &segs[2];
        const int64_t n = 77777;
        s->host.n = n; s->host.index = 2; s->host.offset = 0; s->host.group = &lion;
        s->host.g_dtype = ADAMBRIDGE_DT_BF16; s->host.mv_dtype = ADAMBRIDGE_DT_BF16;
        s->host.out_dtype = ADAMBRIDGE_DT_NONE; s->host.algorithm = ADAMBRIDGE_ALGO_LION;
        s->host.p_dtype = ADAMBRIDGE_DT_F32;
        s->p = new_buf((size_t)n * 4, "seg2 master");
        s->g = new_buf((size_t)n * 2, "seg2 gradient");
        s->m = new_buf((size_t)n * 2, "seg2 m");
        for (int64_t i = 0; i < n; ++i) ((float*)s->p->host)[i] = uniform(-1.0f, 1.0f);
    }
    for (int k = 0; k < 3; ++k) {
        segs[k].dev = segs[k].host;
        attach(&segs[k]);
    }
    for (int b = 0; b < nbufs; ++b) {
        if (upload(&bufs[b])) { fprintf(stderr, "upload of %s failed\n", bufs[b].name); return 2; }
    }

    hipStream_t stream;
    if (hipStreamCreate(&stream) != hipSuccess) { fprintf(stderr, "hipStreamCreate failed\n"); return 2; }
    void* pool = adambridge_pool_create(0, NULL, 0);
    CHECK(pool != NULL, "pool_create: %s", adambridge_last_error());
    if (!pool) return 1;
    CHECK(adambridge_pool_threads(pool) > 0, "pool_threads");
    CHECK(adambridge_pool_set_stream(pool, stream) == 0, "pool_set_stream");

    adambridge_segment* dev[3] = {&segs[0].dev, &segs[1].dev, &segs[2].dev};
    adambridge_segment* host[3] = {&segs[0].host, &segs[1].host, &segs[2].host};
    for (int step = 1; step <= 3; ++step) {
        fill_gradient(&segs[0], 0.0f);
        fill_gradient(&segs[1], 0.001f);
        fill_gradient(&segs[2], 0.01f);
        for (int k = 0; k < 3; ++k) {
            segs[k].host.step = segs[k].dev.step = step;
            if (upload(segs[k].g)) { fprintf(stderr, "gradient upload failed\n"); return 2; }
        }
        int rc = adambridge_multi_step(pool, dev, 3, 0);
        CHECK(rc == 0, "step %d: multi_step returned %d (%s)", step, rc, adambridge_last_error());
        rc = adambridge_pool_sync(pool);
        CHECK(rc == 0, "step %d: pool_sync returned %d (%s)", step, rc, adambridge_last_error());
        rc = oracle_step(host, 3, width, 1);
        CHECK(rc == 0, "step %d: oracle returned %d", step, rc);
        int same = 1;
        for (int b = 0; b < nbufs; ++b) same &= compare(&bufs[b], step);
        printf("step %d: %d buffers %s\n", step, nbufs, same ? "identical to the oracle" : "DIFFER");
        fflush(stdout);

        /* a call with one invalid segment changes nothing (the next step's comparison shows it) */
        adambridge_segment bad = segs[1].dev;
        bad.offset = 100;   /* FP8 chunks start at multiples of 128 */
        adambridge_segment* mixed[2] = {&segs[0].dev, &bad};
        CHECK(adambridge_multi_step(pool, mixed, 2, 0) == ADAMBRIDGE_EOFFSET, "FP8 offset 100 accepted");
    }
    /* multi_apply: explicit coefficients per segment (kernels.c:1630-1641), as the reference's
     * benches and tests call it */
    {
        adambridge_hparams hps[3];
        for (int k = 0; k < 3; ++k) {
            const adambridge_hparams h = {0.85f, 0.98f, 0.15f, 0.02f, 0.999f, 2e-3f * (float)(k + 1), 1.25f, 1e-7f,
                                          0x9e3779b9u * (uint32_t)(k + 11), k != 1};
            hps[k] = h;
        }
        fill_gradient(&segs[0], 0.0f);
        fill_gradient(&segs[1], 0.0f);
        fill_gradient(&segs[2], 0.0f);
        for (int k = 0; k < 3; ++k) {
            if (upload(segs[k].g)) { fprintf(stderr, "gradient upload failed\n"); return 2; }
        }
        int rc = adambridge_multi_apply(pool, dev, hps, 3, 0);
        CHECK(rc == 0, "multi_apply returned %d (%s)", rc, adambridge_last_error());
        CHECK(adambridge_pool_sync(pool) == 0, "pool_sync after multi_apply");
        CHECK(oracle_apply(host, hps, 3, width, 1) == 0, "oracle multi_apply");
        int same = 1;
        for (int b = 0; b < nbufs; ++b) same &= compare(&bufs[b], 4);
        printf("multi_apply: %d buffers %s\n", nbufs, same ? "identical to the oracle" : "DIFFER");
        fflush(stdout);
    }
    /* fused_adamw: one FP32-master tensor with BF16 moments, synchronous (kernels.c:1518-1535);
     * segment 0's buffers at element offset 4099 of a parameter, nearest rounding */
    {
        const adambridge_hparams h = {0.9f, 0.995f, 0.1f, 0.005f, 0.9995f, 1e-3f, 1.5f, 1e-8f, 77u, 0};
        fill_gradient(&segs[0], 0.0f);
        if (upload(segs[0].g)) { fprintf(stderr, "gradient upload failed\n"); return 2; }
        const adambridge_segment* d = &segs[0].dev;
        const int rc = adambridge_fused_adamw((float*)d->p, d->g, d->g_dtype, d->m, d->v, d->mv_dtype, d->out,
                                              d->out_dtype, d->n, 4099, &h);
        CHECK(rc == 0, "fused_adamw returned %d (%s)", rc, adambridge_last_error());
        adambridge_segment o = segs[0].host;
        o.offset = 4099; o.index = 0; o.step = 0; o.group = NULL;
        adambridge_segment* one[1] = {&o};
        CHECK(oracle_apply(one, &h, 1, width, 1) == 0, "oracle fused update");
        int same = 1;
        for (int b = 0; b < nbufs; ++b) same &= compare(&bufs[b], 5);
        printf("fused_adamw: %d buffers %s\n", nbufs, same ? "identical to the oracle" : "DIFFER");
        fflush(stdout);
    }
    CHECK(adambridge_pool_sync(pool) == 0, "final pool_sync");
    adambridge_pool_destroy(pool);
    (void)hipStreamDestroy(stream);
    for (int b = 0; b < nbufs; ++b) {
        (void)hipFree(bufs[b].dev);
        free(bufs[b].host);
    }
    dlclose(lib);
    return failures;
}

int main(int argc, char** argv)
{
    int rc;
    if (argc == 2 && strcmp(argv[1], "abi") == 0) rc = run_abi();
    else if (argc == 3 && strcmp(argv[1], "gpu") == 0) rc = run_gpu(argv[2]);
    else {
        fprintf(stderr, "usage: %s abi | gpu ORACLE.so\n", argv[0]);
        return 2;
    }
    printf("%s (%d failures)\n", rc == 0 ? "PASSED" : "FAILED", failures);
    return rc == 0 ? 0 : 1;
}
