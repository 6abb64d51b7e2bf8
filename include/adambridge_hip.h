/*
 * adambridge_hip.h -- C ABI of libadambridge_hip.so, the fused AdamW / Lion
 * optimizer update for AMD Instinct MI355X (gfx950).
 *
 * Drop-in for the reference's native kernel library, adambridge/csrc/
 * adambridge_kernels.c, as its ctypes binding (adambridge/native.py:273-435)
 * uses it: the same entry-point names, argument meanings, struct layouts,
 * dtype codes and negative error codes.  What changes:
 *
 *   - every buffer pointer in a segment (and in adambridge_fused_adamw) is a
 *     device pointer in HBM of the current HIP device, not a host pointer;
 *   - a "pool" is a launch queue bound to one device and one HIP stream, not
 *     a host thread pool; work is enqueued on that stream and the call returns
 *     once it is enqueued (adambridge_fused_adamw alone waits, as documented);
 *   - the "SIMD level" selects which of the reference's host ISAs is
 *     reproduced bit for bit (its vector bodies fuse multiply-adds, its scalar
 *     tail does not; see adambridge_set_simd_level).
 *
 * All structs, scalars and pointers are plain C; no torch types cross this
 * boundary.  Thread-safety: calls on different pools may run concurrently from
 * different host threads; calls on one pool must not overlap.
 */
#ifndef ADAMBRIDGE_HIP_H
#define ADAMBRIDGE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ADAMBRIDGE_API __attribute__((visibility("default")))

/* ABI version of the reference this library is a drop-in for (kernels.c:71). */
#define ADAMBRIDGE_ABI_VERSION 5

/* Storage codes, kernels.c:73: DT_NONE 0, DT_F32 1, DT_BF16 2, DT_FP8 3, DT_F24 4.
 * Algorithms, kernels.c:75: ALGO_ADAMW 0, ALGO_LION 1.
 * SIMD levels reproduced, kernels.c:74: 0 scalar, 1 AVX2 (8 lanes), 2 AVX-512 (16 lanes). */
enum { ADAMBRIDGE_DT_NONE = 0, ADAMBRIDGE_DT_F32 = 1, ADAMBRIDGE_DT_BF16 = 2, ADAMBRIDGE_DT_FP8 = 3,
       ADAMBRIDGE_DT_F24 = 4, ADAMBRIDGE_DT_PACKED = 5, ADAMBRIDGE_DT_PACKED_FP8 = 6,
       ADAMBRIDGE_DT_PACKED_LION = 7, ADAMBRIDGE_DT_PACKED_F32 = 8, ADAMBRIDGE_DT_PACKED_F24 = 9,
       ADAMBRIDGE_DT_PACKED_LION_F24 = 10, ADAMBRIDGE_DT_PACKED_FP8_F24 = 11, ADAMBRIDGE_DT_PACKED_LION_F32 = 12,
       ADAMBRIDGE_DT_PACKED_LION_FP8 = 13, ADAMBRIDGE_DT_PACKED_F24_F32 = 14, ADAMBRIDGE_DT_PACKED_LION_F24_F32 = 15,
       ADAMBRIDGE_DT_PACKED_LION_FP8_F24 = 16 };

/* ADAMBRIDGE_DT_PACKED (p_dtype; no counterpart in the reference): an HBM layout for
 * AdamW with an FP32 master and BF16 moments (mv_dtype DT_BF16).  p points at 16-byte
 * pairs: for elements 2k and 2k+1 of the segment, {p[2k], p[2k+1] (FP32),
 * m[2k] | m[2k+1] << 16, v[2k] | v[2k+1] << 16 (BF16 bits)}, ceil(n/2) pairs, 16-byte
 * aligned.  m and v are unused.  p_lo is NULL (update in place) or a second buffer of
 * the same layout that receives the new state (double buffering).  Same arithmetic,
 * rounding and rounding streams as the separate layout. */

/* ADAMBRIDGE_DT_PACKED_FP8 (p_dtype; no counterpart in the reference): an HBM layout for
 * AdamW with an FP32 master and FP8 moments (mv_dtype DT_FP8).  p points at one 768-byte
 * record per 128-element block, ceil(n/128) records, 16-byte aligned.  In the record of
 * block b, for l = 0 .. 15, elements 128b + 8l + j hold: master (FP32) at byte 16l + 4j
 * for j < 4 and 256 + 16l + 4(j - 4) for j >= 4; m code (E4M3) at 512 + 16l + j; v code
 * (E5M2, of sqrt v) at 520 + 16l + j.  Elements past n are padding (codes written as 0,
 * master left as it is).  m_scale and v_scale are the usual block scales; m, v and p_lo are
 * unused (p_lo must be NULL).  Same arithmetic, rounding and rounding streams as the
 * separate FP8 layout. */

/* ADAMBRIDGE_DT_PACKED_LION (p_dtype; no counterpart in the reference): an HBM layout for
 * Lion with an FP32 master and a BF16 moment (mv_dtype DT_BF16).  p points at one 1536-byte
 * record per 256 elements, ceil(n/256) records, 16-byte aligned.  The record of elements
 * 256r .. 256r + 255 holds their 256 FP32 masters in element order (bytes 0 .. 1023), then their
 * 256 m values as BF16 bits in element order (bytes 1024 .. 1535).  p_lo is NULL (update in place)
 * or a second buffer of the same layout that receives the new state; m, v and the scales are unused.
 * Slots past n are padding: those up to the end of the last element's group of 4 are written back
 * unchanged (to p_lo, when given), the rest are neither read nor written.  Same arithmetic, rounding and
 * rounding stream as the separate layout. */
/* ADAMBRIDGE_DT_PACKED_LION_F32 (p_dtype; no counterpart in the reference): an HBM layout for
 * Lion with an FP32 master and an FP32 moment (mv_dtype DT_F32).  p points at one 2048-byte
 * record per 256 elements, ceil(n/256) records, 16-byte aligned: the 256 FP32 masters of elements
 * 256r .. 256r + 255 in element order (bytes 0 .. 1023), then their 256 FP32 m values in element
 * order (bytes 1024 .. 2047).  p_lo, padding and arithmetic as in DT_PACKED_LION; the moment is
 * stored exactly (no rounding stream). */
/* ADAMBRIDGE_DT_PACKED_F32 (p_dtype; no counterpart in the reference): an HBM layout for AdamW
 * with an FP32 master and FP32 moments (mv_dtype DT_F32).  p points at one 3072-byte record per
 * 256 elements, ceil(n/256) records, 16-byte aligned.  The record of elements 256r .. 256r + 255
 * holds their 256 masters (bytes 0 .. 1023), then their 256 m values (1024 .. 2047), then their
 * 256 v values (2048 .. 3071), all FP32 in element order.  p_lo is NULL (update in place) or a
 * second buffer of the same layout that receives the new state; m, v and the scales are unused.
 * Padding past n as in DT_PACKED_LION.  Same arithmetic (including the scalar tail's
 * unfused form) as the separate layout. */
/* ADAMBRIDGE_DT_PACKED_F24 (p_dtype; no counterpart in the reference): an HBM layout for AdamW
 * with an FP24 master and BF16 moments (mv_dtype DT_BF16).  p points at one 1792-byte record per
 * 256 elements, ceil(n/256) records, 16-byte aligned.  The record of elements 256r .. 256r + 255
 * holds their 256 master high halves (the FP24 hi plane, BF16 bits; bytes 0 .. 511), then their
 * 256 master low bytes (the lo plane; 512 .. 767), then their 256 m values (768 .. 1279), then
 * their 256 v values (1280 .. 1791), the moments as BF16 bits, everything in element order.
 * p_lo is NULL (update in place) or a second buffer of the same layout that receives the new state;
 * m, v and the scales are unused.  Padding past n as in DT_PACKED_LION.  Same
 * arithmetic, rounding and rounding streams as the separate layout with an FP24 master. */
/* ADAMBRIDGE_DT_PACKED_F24_F32 (p_dtype; no counterpart in the reference): the same for AdamW with an
 * FP24 master and FP32 moments (mv_dtype DT_F32): one 2816-byte record per 256 elements, the 256
 * master high halves (bytes 0 .. 511), the 256 low bytes (512 .. 767), then the 256 m values
 * (768 .. 1791) and the 256 v values (1792 .. 2815) as FP32, everything in element order.  The
 * moments are stored exactly (no rounding streams). */
/* ADAMBRIDGE_DT_PACKED_LION_F24 (p_dtype; no counterpart in the reference): the same for Lion with an
 * FP24 master and a BF16 moment: one 1280-byte record per 256 elements, the 256 master high halves
 * (bytes 0 .. 511), the 256 low bytes (512 .. 767) and the 256 m values (768 .. 1279). */
/* ADAMBRIDGE_DT_PACKED_LION_F24_F32 (p_dtype; no counterpart in the reference): the same with an FP32
 * moment (mv_dtype DT_F32): one 1792-byte record per 256 elements, the m values FP32 at 768 .. 1791,
 * stored exactly. */
/* ADAMBRIDGE_DT_PACKED_FP8_F24 (p_dtype; no counterpart in the reference): an HBM layout for AdamW
 * with an FP24 master and FP8 moments (mv_dtype DT_FP8).  p points at one 640-byte record per
 * 128-element block, ceil(n/128) records, 16-byte aligned.  The record of block b holds its 128
 * master high halves (the FP24 hi plane, BF16 bits; bytes 0 .. 255) and its 128 master low bytes
 * (the lo plane; 256 .. 383), both in element order, then for l = 0 .. 15 the m codes (E4M3) of
 * elements 128b + 8l + j at 384 + 16l + j and their v codes (E5M2, of sqrt v) at 392 + 16l + j.
 * Elements past n are padding (codes written as 0, master left as it is).  m_scale and v_scale are
 * the usual block scales; m, v and p_lo are unused (p_lo must be NULL: updated in place).  Same
 * arithmetic, rounding and rounding streams as the separate FP8 layout with an FP24 master. */
/* ADAMBRIDGE_DT_PACKED_LION_FP8 (p_dtype; no counterpart in the reference): an HBM layout for Lion
 * with an FP32 master and an FP8 moment (mv_dtype DT_FP8).  p points at one 640-byte record per
 * 128-element block, ceil(n/128) records, 16-byte aligned.  The record of block b holds the masters
 * as in DT_PACKED_FP8 (element 128b + 8l + j at byte 16l + 4j for j < 4, 256 + 16l + 4(j - 4) for
 * j >= 4), then the block's 128 m codes (E4M3) in element order (bytes 512 .. 639).  Elements past n
 * are padding (codes written as 0, master left as it is).  m_scale holds the usual block scales;
 * m, v, v_scale and p_lo are unused (p_lo must be NULL: updated in place).  Same arithmetic,
 * rounding and rounding streams as the separate FP8 layout. */
/* ADAMBRIDGE_DT_PACKED_LION_FP8_F24 (p_dtype; no counterpart in the reference): the same for Lion with
 * an FP24 master: one 512-byte record per 128-element block, the master high halves (bytes 0 .. 255)
 * and low bytes (256 .. 383) as in DT_PACKED_FP8_F24, then the block's 128 m codes in element order
 * (384 .. 511). */
enum { ADAMBRIDGE_ALGO_ADAMW = 0, ADAMBRIDGE_ALGO_LION = 1 };

/* Error codes (kernels.c:1537-1553, 1582-1584, 1620-1621), plus the HIP-side ones. */
enum {
    ADAMBRIDGE_OK = 0,
    ADAMBRIDGE_EBADN = -1,         /* negative n, NULL segment array */
    ADAMBRIDGE_ENULL = -2,         /* a required buffer pointer is NULL */
    ADAMBRIDGE_EGDTYPE = -3,
    ADAMBRIDGE_EMVDTYPE = -4,
    ADAMBRIDGE_EOUTDTYPE = -5,
    ADAMBRIDGE_EOUTNULL = -6,
    ADAMBRIDGE_ESCALES = -7,       /* FP8 moments without block scales */
    ADAMBRIDGE_EGROUP = -8,        /* multi_step segment without a group */
    ADAMBRIDGE_ETOOMANY = -9,
    ADAMBRIDGE_ENOMEM = -10,
    ADAMBRIDGE_EOFFSET = -11,      /* negative offset, or FP8 offset not a multiple of 128 */
    ADAMBRIDGE_EALGO = -12,
    ADAMBRIDGE_EPDTYPE = -13,
    ADAMBRIDGE_EALIGN = -14,       /* a packed state buffer is not 16-byte aligned */
    ADAMBRIDGE_EHIP = -20,         /* a HIP runtime call failed; see adambridge_last_error() */
    ADAMBRIDGE_EDEVICE = -21,      /* the pool belongs to another device than the current one */
    ADAMBRIDGE_ECAPTURE = -22      /* a pooled call whose launch needs a staged segment table (more than
                                      7 segments of one kernel variant) on a stream under graph capture */
};

/* Per-segment step coefficients: kernels.c:77-88 (40 bytes). */
typedef struct adambridge_hparams {
    float beta1;
    float beta2;
    float one_minus_beta1;
    float one_minus_beta2;
    float decay;         /* 1 - lr * weight_decay */
    float step_size;     /* AdamW: lr / (1 - beta1^t); Lion: lr */
    float inv_sqrt_bc2;  /* 1 / sqrt(1 - beta2^t) */
    float eps;
    uint32_t seed;       /* rounding stream of this (parameter, step) */
    int32_t stochastic;  /* nonzero: stochastic rounding of BF16/FP8 moments and an FP24 master */
} adambridge_hparams;

/* A parameter group's hyperparameters: kernels.c:736-745 (56 bytes, host memory). */
typedef struct adambridge_group {
    double lr;
    double beta1;
    double beta2;
    double eps;
    double weight_decay;
    uint64_t seed;
    int32_t stochastic;
    int32_t reserved;
} adambridge_group;

/* One tensor (or one chunk of one): kernels.c:747-769 (128 bytes).  The struct
 * itself is host memory; p .. out are device pointers. */
typedef struct adambridge_segment {
    void* p;                 /* FP32 master, the FP24 hi plane (uint16) when p_dtype is DT_F24, or the
                                packed state when p_dtype is DT_PACKED / DT_PACKED_FP8 / DT_PACKED_LION /
                                DT_PACKED_F32 / DT_PACKED_F24 / DT_PACKED_LION_F24 / DT_PACKED_FP8_F24 /
                                DT_PACKED_LION_F32 / DT_PACKED_LION_FP8 / DT_PACKED_F24_F32 /
                                DT_PACKED_LION_F24_F32 / DT_PACKED_LION_FP8_F24 */
    uint8_t* p_lo;           /* FP24 lo plane (one byte per element); NULL for FP32; DT_PACKED,
                                DT_PACKED_LION, DT_PACKED_F32, DT_PACKED_F24, DT_PACKED_LION_F24 and
                                DT_PACKED_LION_F32, DT_PACKED_F24_F32, DT_PACKED_LION_F24_F32: the
                                destination state
                                (NULL: in place) */
    const void* g;           /* gradient, g_dtype */
    void* m;                 /* first moment, mv_dtype (FP8: E4M3 codes, padded to 128 per block) */
    void* v;                 /* second moment (FP8: E5M2 codes of sqrt(v)); unused by Lion */
    float* m_scale;          /* FP8 only: one scale per 128 elements */
    float* v_scale;
    void* out;               /* optional copy of the new master in out_dtype (the bf16 working weight) */
    const adambridge_group* group;   /* multi_step only; host memory */
    int64_t n;
    int64_t step;            /* this update's step number (multi_step) */
    uint64_t index;          /* parameter index: selects the rounding stream */
    int64_t offset;          /* element offset of p[0] within its parameter (multiple of 128 for FP8) */
    int32_t g_dtype;
    int32_t mv_dtype;
    int32_t out_dtype;
    int32_t algorithm;
    int32_t p_dtype;         /* DT_F32 (or 0), DT_F24, DT_PACKED, DT_PACKED_FP8, DT_PACKED_LION, DT_PACKED_F32,
                                DT_PACKED_F24, DT_PACKED_LION_F24, DT_PACKED_FP8_F24, DT_PACKED_LION_F32,
                                DT_PACKED_LION_FP8, DT_PACKED_F24_F32, DT_PACKED_LION_F24_F32 or
                                DT_PACKED_LION_FP8_F24 */
    int32_t reserved;        /* 0, or ADAMBRIDGE_SEG_OUT_PREVIOUS */
} adambridge_segment;

/* ADAMBRIDGE_SEG_OUT_PREVIOUS (a flag in adambridge_segment.reserved; no counterpart in the
 * reference, which leaves the field zero): out receives the working weight of the master as it
 * was stored BEFORE this update -- the value the previous update of the segment wrote to out --
 * instead of the new one.  For updates that reach the weights one step late (delay_updates):
 * the update writes the stale weight straight into the parameter, with no buffer of its own and
 * no copy, and the new weight is the master's, to be written by the next update or a flush.
 * Every other bit of the field is ignored, as the reference ignores the field. */
#define ADAMBRIDGE_SEG_OUT_PREVIOUS 1

/* kernels.c:1493. */
ADAMBRIDGE_API int adambridge_abi_version(void);

/* What this library adds to the reference's ABI version 5 (kept, so that the reference's binding
 * loads it), as bits -- no counterpart in the reference, which has none of these: */
#define ADAMBRIDGE_CAP_PACKED_LAYOUTS 0x01u   /* p_dtype DT_PACKED .. DT_PACKED_LION_F24 (5 .. 10) */
#define ADAMBRIDGE_CAP_OUT_PREVIOUS   0x02u   /* the segment flag ADAMBRIDGE_SEG_OUT_PREVIOUS */
#define ADAMBRIDGE_CAP_NOALLOC        0x04u   /* adambridge_multi_step_noalloc */
#define ADAMBRIDGE_CAP_CONVERT        0x08u   /* adambridge_convert */
#define ADAMBRIDGE_CAP_CONVERT_PLANE  0x10u   /* adambridge_convert_plane */
#define ADAMBRIDGE_CAP_STREAM_COPY    0x20u   /* adambridge_stream_copy, adambridge_recycle_device_memory */
#define ADAMBRIDGE_CAP_FP8_F24_RECORDS 0x40u  /* p_dtype DT_PACKED_FP8_F24 (11) */
#define ADAMBRIDGE_CAP_LION_F32_RECORDS 0x80u /* p_dtype DT_PACKED_LION_F32 (12) */
#define ADAMBRIDGE_CAP_LION_FP8_RECORDS 0x100u /* p_dtype DT_PACKED_LION_FP8 (13); record size in a
                                                 DT_PACKED_FP8 plane's stride */
#define ADAMBRIDGE_CAP_F24_F32_RECORDS 0x200u /* p_dtype DT_PACKED_F24_F32 (14) */
#define ADAMBRIDGE_CAP_LION_F24_F32_RECORDS 0x400u /* p_dtype DT_PACKED_LION_F24_F32 (15) */
#define ADAMBRIDGE_CAP_LION_FP8_F24_RECORDS 0x800u /* p_dtype DT_PACKED_LION_FP8_F24 (16) */
ADAMBRIDGE_API uint32_t adambridge_capabilities(void);

/* kernels.c:1495-1510.  The level whose results are reproduced: its vector
 * body (fused multiply-adds) covers the first n - n mod W elements of every
 * segment and its scalar loop (separately rounded products and sums) the last
 * n mod W, W = 16 at level 2, 8 at level 1; level 0 is the scalar loop for
 * every element.  Lion and FP8 blocks follow the same rule as the reference.
 * Detected level: 2.  set: <0 restores it; returns the level now active.
 * Process-wide, read at enqueue time. */
ADAMBRIDGE_API int adambridge_detected_simd_level(void);
ADAMBRIDGE_API int adambridge_simd_level(void);
ADAMBRIDGE_API int adambridge_set_simd_level(int level);

/* kernels.c:1512-1514: layout checks for bindings. */
ADAMBRIDGE_API int adambridge_hparams_size(void);
ADAMBRIDGE_API int adambridge_group_size(void);
ADAMBRIDGE_API int adambridge_segment_size(void);

/* kernels.c:1518-1535.  One FP32-master AdamW update of n elements with FP32 or
 * BF16 moments, on the calling thread's stream (adambridge_set_stream; the
 * null stream by default).  Waits for completion before returning, like the
 * reference's synchronous call. */
ADAMBRIDGE_API int adambridge_fused_adamw(float* p, const void* g, int g_dtype, void* m, void* v, int mv_dtype,
                                          void* out, int out_dtype, int64_t n, uint64_t offset,
                                          const adambridge_hparams* hp);

/* kernels.c:1427-1487.  A launch queue on the current HIP device, initially on
 * the null stream.  nthreads, cpus and ncpus are accepted and ignored (the
 * device schedules its own compute units).  NULL on failure.  pool_threads
 * returns the device's compute-unit count (1 for a NULL pool, as the
 * reference's); pool_set_spin is a no-op. */
ADAMBRIDGE_API void* adambridge_pool_create(int32_t nthreads, const int32_t* cpus, int32_t ncpus);
ADAMBRIDGE_API void adambridge_pool_destroy(void* pool);
ADAMBRIDGE_API int32_t adambridge_pool_threads(void* pool);
ADAMBRIDGE_API void adambridge_pool_set_spin(void* pool, int32_t spin);

/* kernels.c:1611-1626.  Update every segment; coefficients from its group and
 * step, computed on the host in double as the reference does.  Validates every
 * segment before enqueueing anything (first bad segment's code).  pool NULL:
 * the current device's default queue on the calling thread's stream.
 * threads is ignored.  Asynchronous: ordered on the pool's stream.  Launches
 * are planned in full first (one per kernel variant, split where a variant has
 * more segments than a staging slot holds or more tiles than one dispatch
 * takes), so no size limit is met after something was enqueued.  A launch of
 * more than 7 segments stages its segment table through a reused pinned host
 * slot: on a stream under graph capture such a call returns ADAMBRIDGE_ECAPTURE
 * before enqueueing anything. */
ADAMBRIDGE_API int adambridge_multi_step(void* pool, adambridge_segment* const* segs, int32_t nsegs,
                                         int32_t threads);

/* kernels.c:1630-1641.  As multi_step with caller-supplied coefficients. */
ADAMBRIDGE_API int adambridge_multi_apply(void* pool, adambridge_segment* const* segs,
                                          const adambridge_hparams* hps, int32_t nsegs, int32_t threads);

/* ---- HIP-specific entry points (no counterpart in the reference) ---------- */

/* The HIP stream (a hipStream_t, e.g. torch.cuda.Stream.cuda_stream) on which
 * the pool enqueues from now on.  Returns 0. */
ADAMBRIDGE_API int adambridge_pool_set_stream(void* pool, void* stream);

/* Block until the pool's stream has drained; returns ADAMBRIDGE_EHIP if a
 * kernel of it failed. */
ADAMBRIDGE_API int adambridge_pool_sync(void* pool);

/* The calling thread's stream for pool == NULL calls and adambridge_fused_adamw. */
ADAMBRIDGE_API int adambridge_set_stream(void* stream);

/* Text of the calling thread's last HIP-side failure ("" if none). */
ADAMBRIDGE_API const char* adambridge_last_error(void);

/* Name of the device code this library carries, e.g. "hip/gfx950". */
ADAMBRIDGE_API const char* adambridge_backend(void);

/* adambridge_multi_step with no allocation in the call, for callers that cannot allocate
 * device or pinned memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  No counterpart in the reference.  Same segments, validation, coefficients and
 * results as adambridge_multi_step, enqueued on `stream` (a hipStream_t of the current device;
 * NULL: the null stream).  Instead of a pool's staging buffers it uses one static device array of
 * the library, 152 KiB per GPU, held until the process ends: launches of more than 7 segments of
 * one kernel variant find their segment table there, written by small kernels whose arguments
 * carry the descriptors (no copy from host memory).  Limit: 1024 segments per call (more:
 * ADAMBRIDGE_ETOOMANY, with the reason in adambridge_last_error(), before anything is enqueued).
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU (other streams,
 * other threads, or replays of graphs holding such calls) race and must be ordered by the caller;
 * calls from several host threads are serialised on the host.  ADAMBRIDGE_EDEVICE if the stream
 * belongs to another device. */
ADAMBRIDGE_API int adambridge_multi_step_noalloc(void* stream, adambridge_segment* const* segs, int32_t nsegs);

/* The launches a multi_apply / multi_step call over these segments would make, without
 * launching anything or touching the device (a diagnostic for bindings and tests).  Segments are
 * validated as multi_apply validates them.  For each entry of each launch, in launch order, writes
 * four values to rows[4k .. 4k + 3] while k < cap: the launch's number, its kernel variant, the
 * entry's first tile (negative where a segment continues from the previous launch) and the
 * launch's tile count.  A segment appears once, or once per launch its tiles are spread over when
 * they exceed one dispatch (2^32 - 1 work-items).  Returns the number of entries (which may
 * exceed cap), or a negative code. */
ADAMBRIDGE_API int adambridge_plan_launches(adambridge_segment* const* segs, int32_t nsegs, int64_t* rows,
                                            int32_t cap);

/* Re-encodes n values of one moment (role 0: m, FP8 as E4M3FN; role 1: v, FP8 as E5M2 of
 * sqrt(v)) or of an FP32 master (role 0) from src_dtype to dst_dtype (ADAMBRIDGE_DT_F32, _BF16 or
 * _FP8), on the calling thread's stream (asynchronous).  The device form of the conversions the
 * reference's stores make with torch when precision or a checkpoint's format changes
 * (precision.py:341-418, 555-575; engine.py:1030-1043): values decoded exactly, then encoded to
 * nearest -- BF16, or FP8 per 128-element block with scale = absmax / format max (1 for an
 * all-zero block or one holding a NaN), v in the sqrt domain after clamping at zero.  FP8 buffers
 * hold codes padded to whole blocks (all written) and one scale per block.  Returns 0,
 * ADAMBRIDGE_EBADN (n < 0), _EMVDTYPE (unknown dtype or role), _ENULL, _ESCALES (FP8 without its
 * scales) or _EHIP (launch failure). */
ADAMBRIDGE_API int adambridge_convert(const void* src, const float* src_scale, int32_t src_dtype, void* dst,
                                      float* dst_scale, int32_t dst_dtype, int64_t n, int32_t role);

/* One plane of values in device memory, for adambridge_convert_plane (no counterpart in the
 * reference).  Element i of the plane is the value at
 *     data + (i >> group_log2) * stride + (i mod 2^group_log2) * size,
 * size being 4 bytes (ADAMBRIDGE_DT_F32) or 2 (ADAMBRIDGE_DT_BF16: BF16 bits; ADAMBRIDGE_DT_F24:
 * the high half, with the low byte at lo + (i >> group_log2) * stride + (i mod 2^group_log2)).
 * stride 0: contiguous (group_log2 unused).  ADAMBRIDGE_DT_PACKED_FP8: the FP32 masters of FP8
 * block records at data (the layout above), stride the record size: 768 (or 0) for DT_PACKED_FP8
 * records, 640 for DT_PACKED_LION_FP8 (group_log2 unused).  The masters of the other
 * interleaved layouts at a state buffer s are the planes
 *     DT_PACKED           {s, NULL, 16, DT_F32, 1}       DT_PACKED_LION      {s, NULL, 1536, DT_F32, 8}
 *     DT_PACKED_F32       {s, NULL, 3072, DT_F32, 8}     DT_PACKED_F24       {s, s + 512, 1792, DT_F24, 8}
 *     DT_PACKED_LION_F24  {s, s + 512, 1280, DT_F24, 8}   DT_PACKED_LION_F32  {s, NULL, 2048, DT_F32, 8}
 *     DT_PACKED_F24_F32   {s, s + 512, 2816, DT_F24, 8}   DT_PACKED_LION_F24_F32 {s, s + 512, 1792, DT_F24, 8}
 *     DT_PACKED_FP8_F24   {s, s + 256, 640, DT_F24, 7}    DT_PACKED_LION_FP8_F24 {s, s + 256, 512, DT_F24, 7}
 * and a separate FP24 master is {hi, lo, 0, DT_F24, 0}.  data is aligned to its value size (16 bytes
 * for DT_PACKED_FP8) and stride a multiple of it. */
typedef struct adambridge_plane {
    void* data;
    uint8_t* lo;
    int64_t stride;
    int32_t dtype;
    int32_t group_log2;
} adambridge_plane;

#define ADAMBRIDGE_CONVERT_STOCHASTIC 1

/* No counterpart in the reference; the device form of the FP24 master's conversions
 * (precision.py:421-480: rounding FP32 values into the planes, expanding them back) and of the
 * working weight a master gives (kernels.c:108-112).  Copies n values from plane src to plane dst on
 * the calling thread's stream (asynchronous), converting between the planes' types: a value that
 * the destination type represents (BF16 into FP24 or FP32, FP24 into FP32, any type into itself) is
 * copied bit for bit, NaN payloads included; otherwise it is rounded as the kernels round it --
 * into BF16 to nearest even with a NaN quietened (sign and payload kept), into FP24 to nearest even
 * on the top 24 bits with a NaN quietened (kernels.c:145-160) -- or, with flags
 * ADAMBRIDGE_CONVERT_STOCHASTIC, stochastically: element i adds the low 16 (BF16) or 8 (FP24) bits
 * of lowbias32(uint32(offset + i) ^ seed) before the cut (kernels.c:120-126, 145-150; seed is the
 * stream's 32-bit seed itself).  src and dst must not overlap unless they are the same plane.
 * Returns 0, ADAMBRIDGE_EBADN (n < 0, unknown flags, a negative stride or a group_log2 outside
 * 0 .. 30), _ENULL (a NULL plane, data, or FP24 lo), _EPDTYPE (a type other than those above),
 * _EALIGN or _EHIP (launch failure). */
ADAMBRIDGE_API int adambridge_convert_plane(const adambridge_plane* src, const adambridge_plane* dst, int64_t n,
                                            uint64_t offset, uint32_t seed, int32_t flags);

/* No counterpart in the reference: allocates nbytes of device memory on the current device and
 * frees it at once.  For callers about to allocate a large buffer that the fused update streams
 * (the optimizer's state arena): on MI355X the first allocations a fresh process gets from the
 * driver land where the update streams ~3-4% slower than a copy, while an allocation that follows
 * an allocate/free of its own size lands where it streams at the copy's rate (measured on the 7B
 * bf16-moment step: 21.43 against 20.75 ms per launch, first build of a fresh process).  Peak
 * memory is nbytes.  0, ADAMBRIDGE_EBADN (nbytes < 0) or ADAMBRIDGE_EHIP (the allocation failed:
 * nothing is held and the HIP error is cleared). */
ADAMBRIDGE_API int adambridge_recycle_device_memory(int64_t nbytes);

/* Copies nbytes (a multiple of 16; src and dst 16-byte aligned, not overlapping) on the calling
 * thread's stream with the update kernels' access type -- 16-byte non-temporal global loads and
 * stores, 4 KiB workgroup tiles handed out XCD by XCD, at most 6 workgroups per CU (kernel
 * k_stream_copy, one launch per 64 GiB) -- so that hardware byte counters (rocprofv3 FETCH_SIZE / WRITE_SIZE) read for it calibrate the
 * same counters read for the update kernels, and its time bounds what a 1:1 read/write stream of
 * the same bytes reaches.  Asynchronous.  Returns 0, ADAMBRIDGE_EBADN (negative or not a multiple of
 * 16), _ENULL, _EALIGN or _EHIP.  No counterpart in the reference: a measurement aid. */
ADAMBRIDGE_API int adambridge_stream_copy(const void* src, void* dst, int64_t nbytes);

/* Self-check of the device's conversion, square-root and reciprocal instructions, on the current
 * device (synchronous).  The kernels round to FP8 and BF16 with gfx950's conversion instructions
 * wherever those give the reference's codes (kernels.c:108-112, 857-876), and take square roots
 * and FP8 block reciprocals with short sequences where they are correctly rounded; this runs every
 * FP32 bit pattern through them and through integer forms of the reference's rules (sqrtf), in
 * those ranges, with random bits hash32(x ^ seed) for the stochastic ones.  Writes min(count, 9)
 * counts of differing results:
 * [0] stochastic E4M3, [1] stochastic E5M2, [2] nearest-even E4M3, [3] nearest-even E5M2,
 * [4] BF16 nearest-even, [5] square roots -- sqrtf on every finite x >= 0, and the short form
 * (v_sqrt_f32 and one Newton correction with v_rsq_f32) on 2^-100 <= x < 2^100 -- against the nearest root
 * decided in exact integer arithmetic, [6] FP8 decoding of every code of
 * both formats against the formats' definitions, [7] divisions -- 2^32 sampled pairs of the
 * AdamW step's m / den and of the FP8 block quotients -- against the nearest quotient in exact
 * integer arithmetic, [8] reciprocals -- the short form (v_rcp_f32 and one Newton step) on every
 * 2^-126 <= s < 2^126 -- against the nearest quotient 1 / s in exact integer arithmetic -- all
 * zero on a conforming device.
 * Returns the number of checks (9),
 * ADAMBRIDGE_ENULL for a NULL array or count < 1, ADAMBRIDGE_EHIP on a HIP failure. */
ADAMBRIDGE_API int adambridge_check_conversions(uint32_t seed, uint64_t* mismatches, int32_t count);

#ifdef __cplusplus
}
#endif

#endif /* ADAMBRIDGE_HIP_H */
