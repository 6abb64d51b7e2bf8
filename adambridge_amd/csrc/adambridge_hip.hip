// adambridge_hip.hip -- fused AdamW / Lion optimizer update for MI355X (gfx950)
// and the C ABI declared in include/adambridge_hip.h.
//
// One launch updates every segment (tensor) of a call: the grid is a list of
// tiles of L.tile elements, each workgroup finds its segment by a binary search
// of the per-segment first-tile table (uniform, scalar loads), then streams its
// tile once: reads the gradient, the master and the moments, updates them in
// registers and writes the master, the moments and the bf16 working weight.
// Non-temporal global loads and stores, one pass: the bytes moved per element
// are exactly the reference's minimum (benchmarks/bench_kernels.py:63-65).
//
// Tiles are small (1024 elements for the FP32/BF16-moment kernels) and handed
// out XCD by XCD: the hardware deals consecutive workgroups round-robin to the
// 8 XCDs, so workgroup b takes tile (b mod 8) * ceil(ntiles/8) + b / 8 and each
// XCD sweeps one contiguous eighth of the launch.  The accesses in flight then
// cover a few compact address windows, which HBM serves with far fewer row
// switches than the scattered windows of large per-workgroup tiles (measured on
// MI355X: a 1:1 read/write stream goes from 5.4 to 6.5 TB/s).
//
// FP8 moments are handled 128-element block by block: 16 lanes x 8 elements
// per block (one DPP row), the two block maxima reduced by DPP row maxima, codes and
// scales written by the same lanes (kernels.c:1034-1059).  In the block-record layout
// (DT_PACKED8) a block's master and both code arrays are one 768-byte record, read
// and written with three 16-byte accesses per lane; Lion's (DT_PACKED8_LION) is a
// 640-byte record of the same masters and the m codes (two 16-byte and one 8-byte access).
//
// Segment descriptors travel in the kernel arguments when a call has at most
// kInline segments (the per-parameter hook path: no copy at all), otherwise in
// a device table filled by one asynchronous copy from a pinned staging slot.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <mutex>
#include <utility>
#include <new>
#include <vector>

#include "../../include/adambridge_hip.h"
#include "abh_device.hpp"

namespace abh {

constexpr int kThreads = 256;
// Elements per workgroup: a launch parameter, a multiple of the kernel family's quantum -- one
// pass of the 256 lanes (two elements each) of the FP32/BF16-moment kernels, or of the 16 block
// groups (128 elements each) of the FP8 kernel.
constexpr int64_t kPairQuantum = 2 * kThreads;
constexpr int64_t kFp8Quantum = (kThreads / 16) * kFp8Block;
constexpr int kInline = 7;        // segments carried in the kernel arguments

// Address spaces: buffers are global memory, descriptors are read-only and uniform (scalar loads).
#define ABH_GLOBAL __attribute__((address_space(1)))
#define ABH_CONST __attribute__((address_space(4)))

// Per-segment launch descriptor (device side), 144 bytes.
struct DevSeg {
    void* p;
    uint8_t* p_lo;
    const void* g;
    void* m;
    void* v;
    float* m_scale;
    float* v_scale;
    void* out;
    int64_t n;
    int64_t n_main;      // [0, n_main) take the fused form, [n_main, n) the scalar-tail form
    int64_t tile_begin;  // first tile of this segment in the launch
    uint32_t idx0;       // uint32(offset): element i draws rounding bits at idx0 + i
    uint32_t flags;      // kVec: every pointer allows 16-byte access; kSR: stochastic rounding;
                         // kPrev: out receives the weight of the master before the update;
                         // kFastDiv: the coefficients allow quot_fast (adamw8_fused)
    Coef c;
    uint32_t seed_m, seed_v, seed_p, pad;
};
static_assert(sizeof(DevSeg) == 144, "DevSeg layout");
constexpr uint32_t kVec = 1u, kSR = 2u, kPrev = 4u, kFastDiv = 8u;

struct Launch {
    const DevSeg* table;     // device table when nsegs > kInline
    const int64_t* starts;   // device: first tile of each segment (compact, for the search)
    int64_t tile;            // elements per tile (multiple of the kernel family's quantum)
    int64_t ntiles;          // tiles of the launch; the grid is ntiles rounded up to a multiple of 8
    int32_t nsegs;
    int32_t pad;
    DevSeg inl[kInline];
};
static_assert(sizeof(Launch) <= 1024 + 64, "kernel argument block");

constexpr int kXcds = 8;

// The tile of this workgroup (XCD-contiguous order, see the file comment); >= L.ntiles for the
// few workgroups that round the grid up to a multiple of 8.
__device__ __forceinline__ int64_t block_tile(const Launch& L)
{
    const int64_t b = blockIdx.x;
    const int64_t per = (L.ntiles + kXcds - 1) / kXcds;
    return (b % kXcds) * per + b / kXcds;
}

// A descriptor copied word by word out of the constant address space (scalar loads).
__device__ __forceinline__ DevSeg load_desc(const ABH_CONST DevSeg* p)
{
    constexpr int kWords = sizeof(DevSeg) / 8;
    union { DevSeg s; uint64_t w[kWords]; } u;
    const ABH_CONST uint64_t* q = (const ABH_CONST uint64_t*)p;
#pragma unroll
    for (int k = 0; k < kWords; ++k) u.w[k] = q[k];
    return u.s;
}

// The descriptor of the segment holding `tile`: binary search of the first-tile table, all
// through scalar loads (uniform address, constant address space), result in scalar registers.
__device__ __forceinline__ DevSeg find_segment(const Launch& L, int64_t tile)
{
    int lo = 0, hi = L.nsegs - 1;
    if (L.nsegs <= kInline) {
        const ABH_CONST DevSeg* inl = (const ABH_CONST DevSeg*)&L.inl[0];
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (inl[mid].tile_begin <= tile) lo = mid; else hi = mid - 1;
        }
        return load_desc(inl + lo);
    }
    const ABH_CONST int64_t* starts = (const ABH_CONST int64_t*)L.starts;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (starts[mid] <= tile) lo = mid; else hi = mid - 1;
    }
    return load_desc((const ABH_CONST DevSeg*)L.table + lo);
}

// --------------------------------------------------------------- loads/stores

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Streaming accesses: every byte is touched once per step, so keep them out of the caches.
// The casts make them global_load / global_store (not flat): the buffers are device memory.
template <typename T>
__device__ __forceinline__ T ld(const T* p) { return __builtin_nontemporal_load((const ABH_GLOBAL T*)p); }
template <typename T>
__device__ __forceinline__ void st(T* p, T v) { __builtin_nontemporal_store(v, (ABH_GLOBAL T*)p); }

// A lane's address: a uniform byte offset from a buffer plus a 32-bit per-lane offset.  The
// uniform part stays in scalar registers and the access takes the global instructions' scalar-base
// form (one 32-bit vector offset), with no 64-bit address arithmetic per lane.
template <typename T>
__device__ __forceinline__ T* lane_ptr(const void* base, int64_t ubytes, uint32_t lane)
{
    char* const u = static_cast<char*>(const_cast<void*>(base)) + ubytes;
    return reinterpret_cast<T*>(u + lane);
}

// The same 32-bit lane offset as a new value: an address formed from it is formed where it is
// used.  Instruction selection sees one basic block at a time, so an address computed before a
// branch and used after it reaches the store as a 64-bit vector value, which loses the
// scalar-base form.
__device__ __forceinline__ uint32_t fresh(uint32_t x)
{
    asm volatile("" : "+v"(x));
    return x;
}

// 8 BF16 values, two to a word (element 2k in the low half of word k), as FP32.
__device__ __forceinline__ void decode_bf16x8(const u32x4 w, float (&x)[8])
{
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        x[2 * k] = bitsf(u[k] << 16);
        x[2 * k + 1] = bitsf(u[k] & 0xffff0000u);
    }
}

// 8 FP24 values from their planes (high halves two to a word, low bytes four to a word) as FP32:
// value k = high half k & 1 of word k >> 1 : low byte k & 3 of word k >> 2 : a zero byte, one byte
// permute each (selector bytes 4-7 address the first source, 0-3 the second, 0x0c gives zero).
__device__ __forceinline__ void decode_f24x8(const u32x4 h, const u32x2 l, float (&x)[8])
{
    const uint32_t hu[4] = {h.x, h.y, h.z, h.w};
    const uint32_t lu[2] = {l.x, l.y};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t hb = 4u + 2u * (uint32_t)(k & 1);
        const uint32_t sel = 0x0cu | (uint32_t)(k & 3) << 8 | hb << 16 | (hb + 1u) << 24;
        x[k] = bitsf(__builtin_amdgcn_perm(hu[k >> 1], lu[k >> 2], sel));
    }
}

// 8 consecutive values at p as FP32, from BF16 bits or FP32, 16-byte aligned.
template <int DT>
__device__ __forceinline__ void load8(const void* p, float (&x)[8])
{
    if constexpr (DT == DT_BF16) {
        decode_bf16x8(ld(static_cast<const u32x4*>(p)), x);
    } else {
        // Two 16-byte loads per lane at a 32-byte lane stride: each load covers half of every cache
        // line it touches.  Ordinary (cached) loads let the second find the line the first brought
        // into L2; non-temporal ones fetched most lines twice (measured: 1.39x the FP8 kernel's
        // algorithmic reads, 8% slower).
        const f32x4* q = static_cast<const f32x4*>(p);
        const f32x4 a = *(const ABH_GLOBAL f32x4*)q, b = *(const ABH_GLOBAL f32x4*)(q + 1);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    }
}

__device__ __forceinline__ void store8_f32(void* p, const float (&x)[8])
{
    f32x4* q = static_cast<f32x4*>(p);
    st(q, f32x4{x[0], x[1], x[2], x[3]});
    st(q + 1, f32x4{x[4], x[5], x[6], x[7]});
}

// Master: FP32, or FP24 = hi plane (BF16 bits) << 16 | lo plane << 8.
// FP8 records (p_dtype DT_PACKED8): the FP32 master and both FP8 moments of a 128-element block
// in one 768-byte record, in the FP8 kernel's lane order.  Lane l of the block's 16 holds
// elements 8l .. 8l + 7: their master at byte 16l (elements 8l .. 8l + 3) and 256 + 16l
// (8l + 4 .. 8l + 7), their E4M3 m codes at 512 + 16l and E5M2 v codes at 520 + 16l.  Each of
// the lane's three 16-byte accesses is one contiguous 256-byte span per block.
constexpr int64_t kRecordBytes = 768;

// Lion FP8 records (p_dtype DT_PACKED8_LION): the FP32 master and the m codes of a 128-element block
// in one 640-byte record, the masters as in DT_PACKED8 (bytes 0 .. 511) and the block's 128 E4M3 codes
// in element order at 512 (lane l's 8 at 512 + 8l).  Lane l's three accesses (two 16-byte master
// halves, 8 bytes of codes) are each one contiguous span per block.
constexpr int64_t kRecordBytesLion8 = 640;

// Byte offset of element i's master value within records of rec bytes (768 or 640).
__device__ __forceinline__ int64_t record_master_offset(int64_t i, int64_t rec = kRecordBytes)
{
    return (i >> 7) * rec + ((i & 4) ? 256 : 0) + ((i >> 3) & 15) * 16 + (i & 3) * 4;
}

// FP8 records with an FP24 master (p_dtype DT_PACKED8_F24): per 128-element block one 640-byte record,
// the block's master high halves (bytes 0 .. 255) and low bytes (256 .. 383) in element order, then
// lane l's m codes at 384 + 16l and v codes at 392 + 16l, as in DT_PACKED8.  Lane l's three
// accesses (16-byte high halves, 8-byte low bytes, 16-byte codes) are each one contiguous span per
// block.
constexpr int64_t kRecordBytesF24 = 640;

// Byte offsets of element i's master high half and low byte within those records.
// Lion FP8 records with an FP24 master (p_dtype DT_PACKED8_LION_F24) are the same without the v codes:
// 512 bytes, lane l's m codes at 384 + 8l (the block's codes in element order).
constexpr int64_t kRecordBytesLion8F24 = 512;

__device__ __forceinline__ int64_t record_f24_hi_offset(int64_t i, int64_t rec = kRecordBytesF24)
{
    return (i >> 7) * rec + (i & 127) * 2;
}
__device__ __forceinline__ int64_t record_f24_lo_offset(int64_t i, int64_t rec = kRecordBytesF24)
{
    return (i >> 7) * rec + 256 + (i & 127);
}

// The masters of 8 consecutive elements: the FP24 planes at p (high halves) and lo (low bytes),
// a record's two 16-byte halves at p and p + 256 (DT_PACKED8), or FP32 at p.
template <int PT>
__device__ __forceinline__ void load_master8(const void* p, const uint8_t* lo, float (&x)[8])
{
    if constexpr (PT == DT_F24) {
        decode_f24x8(ld(static_cast<const u32x4*>(p)), ld(reinterpret_cast<const u32x2*>(lo)), x);
    } else if constexpr (PT == DT_PACKED8) {
        const uint8_t* r = static_cast<const uint8_t*>(p);
        const f32x4 a = ld(reinterpret_cast<const f32x4*>(r)), b = ld(reinterpret_cast<const f32x4*>(r + 256));
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    } else {
        load8<DT_F32>(p, x);
    }
}

// Rounds and stores 8 new master values (at p and lo, as load_master8); x becomes the values
// stored.  idx % 8 == 0 (the FP8 kernel's lanes start at multiples of 8 within segments that start
// at multiples of 128), so idx + k == idx ^ k and the 8 rounding draws share one hash head.
template <int PT, bool SR>
__device__ __forceinline__ void store_master8(void* p, uint8_t* lo, float (&x)[8], uint32_t idx, uint32_t seed,
                                              const Wave8& w)
{
    if constexpr (PT == DT_F24) {
        uint32_t r[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
        if constexpr (SR) hash8_low8(idx, seed, w, r);   // f24_round takes r & 0xff
        // f24_round: the add and the cut, and a NaN quietened instead; the NaN fix-up runs only
        // where some lane of the wavefront holds one (a uniform test: the lane's 8 values through
        // gfx950's NaN-keeping three-operand maximum, v_maximum3_f32, then one compare)
        float any = x[0];
        uint32_t b[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if (k > 0) any = __builtin_elementwise_maximum(any, x[k]);
            const uint32_t u = fbits(x[k]);
            b[k] = (SR ? u + r[k] : u + 0x7fu + ((u >> 8) & 1u)) & ~0xffu;   // r[k] < 256
        }
        if (__builtin_amdgcn_ballot_w64(any != any) != 0) {
#pragma unroll
            for (int k = 0; k < 8; ++k) b[k] = f24_round<SR>(x[k], r[k]);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) x[k] = bitsf(b[k]);
        // the planes by byte permutes: high halves two to a word, low bytes four to a word
        const u32x4 h = {__builtin_amdgcn_perm(b[1], b[0], 0x07060302u), __builtin_amdgcn_perm(b[3], b[2], 0x07060302u),
                         __builtin_amdgcn_perm(b[5], b[4], 0x07060302u), __builtin_amdgcn_perm(b[7], b[6], 0x07060302u)};
        const u32x2 l = {__builtin_amdgcn_perm(b[1], b[0], 0x0c0c0501u) | __builtin_amdgcn_perm(b[3], b[2], 0x05010c0cu),
                         __builtin_amdgcn_perm(b[5], b[4], 0x0c0c0501u) | __builtin_amdgcn_perm(b[7], b[6], 0x05010c0cu)};
        st(static_cast<u32x4*>(p), h);
        st(reinterpret_cast<u32x2*>(lo), l);
    } else if constexpr (PT == DT_PACKED8) {
        uint8_t* r = static_cast<uint8_t*>(p);
        st(reinterpret_cast<f32x4*>(r), f32x4{x[0], x[1], x[2], x[3]});
        st(reinterpret_cast<f32x4*>(r + 256), f32x4{x[4], x[5], x[6], x[7]});
    } else {
        store8_f32(p, x);
    }
}

template <int OT>
__device__ __forceinline__ void store_out8(void* p, const float (&x)[8])
{
    if constexpr (OT == DT_BF16) {
        const u32x4 w = {bf16x2_rne(x[0], x[1]), bf16x2_rne(x[2], x[3]), bf16x2_rne(x[4], x[5]),
                         bf16x2_rne(x[6], x[7])};
        st(static_cast<u32x4*>(p), w);
    } else if constexpr (OT == DT_F32) {
        store8_f32(p, x);
    }
}

// ------------------------------------------------ two elements per lane
//
// The FP32/BF16-moment kernel gives each lane two consecutive elements: one
// small access per buffer per lane.  Measured on MI355X this streams faster
// than wider per-lane chunks (fewer bytes in flight per lane to distinct rows).

template <int DT>
__device__ __forceinline__ void load2(const void* base, int64_t i, float& x0, float& x1)
{
    if constexpr (DT == DT_BF16) {
        const uint32_t w = ld(reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(base) + i));
        x0 = bitsf(w << 16);
        x1 = bitsf(w & 0xffff0000u);
    } else {
        const f32x2 w = ld(reinterpret_cast<const f32x2*>(static_cast<const float*>(base) + i));
        x0 = w.x;
        x1 = w.y;
    }
}

__device__ __forceinline__ void store2_f32(void* base, int64_t i, float x0, float x1)
{
    st(reinterpret_cast<f32x2*>(static_cast<float*>(base) + i), f32x2{x0, x1});
}

__device__ __forceinline__ void store2_u16(void* base, int64_t i, uint32_t h0, uint32_t h1)
{
    st(reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(base) + i), h0 | (h1 << 16));
}

template <int PT>
__device__ __forceinline__ void load_master2(const DevSeg& s, int64_t i, float& x0, float& x1)
{
    if constexpr (PT == DT_F24) {
        const uint32_t h = ld(reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(s.p) + i));
        const uint32_t l = ld(reinterpret_cast<const uint16_t*>(s.p_lo + i));
        x0 = bitsf((h << 16) | ((l & 0xffu) << 8));
        x1 = bitsf((h & 0xffff0000u) | (l & 0xff00u));
    } else {
        load2<DT_F32>(s.p, i, x0, x1);
    }
}

// Rounds and stores two new master values; x0, x1 become the values stored.
template <int PT, bool SR>
__device__ __forceinline__ void store_master2(const DevSeg& s, int64_t i, float& x0, float& x1, uint32_t idx)
{
    if constexpr (PT == DT_F24) {
        const uint32_t b0 = f24_round<SR>(x0, SR ? hash32(idx ^ s.seed_p) : 0u);
        const uint32_t b1 = f24_round<SR>(x1, SR ? hash32((idx + 1) ^ s.seed_p) : 0u);
        x0 = bitsf(b0);
        x1 = bitsf(b1);
        st(reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(s.p) + i), (b0 >> 16) | (b1 & 0xffff0000u));
        st(reinterpret_cast<uint16_t*>(s.p_lo + i), (uint16_t)(((b0 >> 8) & 0xffu) | (b1 & 0xff00u)));
    } else {
        store2_f32(s.p, i, x0, x1);
    }
}

template <int MV, bool SR>
__device__ __forceinline__ void store_moment2(void* base, int64_t i, float x0, float x1, uint32_t idx, uint32_t seed)
{
    if constexpr (MV == DT_BF16) {
        store2_u16(base, i, bf16_store<SR>(x0, SR ? hash32(idx ^ seed) : 0u),
                   bf16_store<SR>(x1, SR ? hash32((idx + 1) ^ seed) : 0u));
    } else {
        store2_f32(base, i, x0, x1);
    }
}

template <int OT>
__device__ __forceinline__ void store_out2(void* base, int64_t i, float x0, float x1)
{
    if constexpr (OT == DT_BF16) st(reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(base) + i), bf16x2_rne(x0, x1));
    else if constexpr (OT == DT_F32) store2_f32(base, i, x0, x1);
}

// ------------------------------------------------------------ scalar access

template <int DT>
__device__ __forceinline__ float load1(const void* base, int64_t i)
{
    if constexpr (DT == DT_BF16) return bitsf((uint32_t)ld(static_cast<const uint16_t*>(base) + i) << 16);
    else return ld(static_cast<const float*>(base) + i);
}

template <int PT>
__device__ __forceinline__ float load_master1(const DevSeg& s, int64_t i)
{
    if constexpr (PT == DT_F24)
        return bitsf(((uint32_t)ld(static_cast<const uint16_t*>(s.p) + i) << 16) | ((uint32_t)ld(s.p_lo + i) << 8));
    else if constexpr (PT == DT_PACKED8_F24 || PT == DT_PACKED8_LION_F24) {
        constexpr int64_t rec = PT == DT_PACKED8_F24 ? kRecordBytesF24 : kRecordBytesLion8F24;
        const uint8_t* r = static_cast<const uint8_t*>(s.p);
        return bitsf(((uint32_t)ld(reinterpret_cast<const uint16_t*>(r + record_f24_hi_offset(i, rec))) << 16) |
                     ((uint32_t)ld(r + record_f24_lo_offset(i, rec)) << 8));
    } else if constexpr (PT == DT_PACKED8 || PT == DT_PACKED8_LION)
        return ld(reinterpret_cast<const float*>(static_cast<const uint8_t*>(s.p) +
                                                 record_master_offset(i, PT == DT_PACKED8 ? kRecordBytes : kRecordBytesLion8)));
    else return ld(static_cast<const float*>(s.p) + i);
}

template <int PT, bool SR>
__device__ __forceinline__ float store_master1(const DevSeg& s, int64_t i, float x, uint32_t idx)
{
    if constexpr (PT == DT_F24) {
        const uint32_t b = f24_round<SR>(x, SR ? hash32(idx ^ s.seed_p) : 0u);
        st(static_cast<uint16_t*>(s.p) + i, (uint16_t)(b >> 16));
        st(s.p_lo + i, (uint8_t)(b >> 8));
        return bitsf(b);
    } else if constexpr (PT == DT_PACKED8_F24 || PT == DT_PACKED8_LION_F24) {
        constexpr int64_t rec = PT == DT_PACKED8_F24 ? kRecordBytesF24 : kRecordBytesLion8F24;
        const uint32_t b = f24_round<SR>(x, SR ? hash32(idx ^ s.seed_p) : 0u);
        uint8_t* r = static_cast<uint8_t*>(s.p);
        st(reinterpret_cast<uint16_t*>(r + record_f24_hi_offset(i, rec)), (uint16_t)(b >> 16));
        st(r + record_f24_lo_offset(i, rec), (uint8_t)(b >> 8));
        return bitsf(b);
    } else if constexpr (PT == DT_PACKED8 || PT == DT_PACKED8_LION) {
        st(reinterpret_cast<float*>(static_cast<uint8_t*>(s.p) +
                                    record_master_offset(i, PT == DT_PACKED8 ? kRecordBytes : kRecordBytesLion8)), x);
        return x;
    } else {
        st(static_cast<float*>(s.p) + i, x);
        return x;
    }
}

template <int MV, bool SR>
__device__ __forceinline__ void store_moment1(void* base, int64_t i, float x, uint32_t r)
{
    if constexpr (MV == DT_BF16) st(static_cast<uint16_t*>(base) + i, (uint16_t)bf16_store<SR>(x, r));
    else st(static_cast<float*>(base) + i, x);
}

template <int OT>
__device__ __forceinline__ void store_out1(void* base, int64_t i, float x)
{
    if constexpr (OT == DT_BF16) st(static_cast<uint16_t*>(base) + i, (uint16_t)bf16_rne(x));
    else if constexpr (OT == DT_F32) st(static_cast<float*>(base) + i, x);
}

// ------------------------------------------------- FP32 / BF16 moment kernel

// ALGO: AdamW or Lion; MV: moment storage (F32 / BF16); PT: master (F32 / F24);
// GT: gradient (F32 / BF16); OT: working-weight output (NONE / F32 / BF16);
// SR: stochastic rounding of BF16 moments and an FP24 master.
template <int ALGO, int MV, int PT, int GT, int OT, bool SR>
__device__ __forceinline__ void update_tile(const DevSeg& s, int64_t tile, int64_t T)
{
    const int64_t n = s.n, n_main = s.n_main;
    const int64_t lo = (tile - s.tile_begin) * T;
    const int64_t hi = lo + T < n ? lo + T : n;
    const Coef c = s.c;
    const int64_t nvec = (s.flags & kVec) ? (n_main & ~(int64_t)1) : 0;
    const bool prev = (s.flags & kPrev) != 0;   // uniform: out from the master as loaded
    int64_t vend = hi < nvec ? hi : nvec;
    if (vend < lo) vend = lo;

    // each workgroup streams one contiguous tile: pairs of elements, both in the fused range
    for (int64_t i = lo + threadIdx.x * 2; i < vend; i += kThreads * 2) {
        const uint32_t idx = s.idx0 + (uint32_t)i;
        float g0, g1, m0, m1, v0 = 0.0f, v1 = 0.0f, p0, p1;
        load2<GT>(s.g, i, g0, g1);
        load2<MV>(s.m, i, m0, m1);
        if constexpr (ALGO == ALGO_ADAMW) load2<MV>(s.v, i, v0, v1);
        load_master2<PT>(s, i, p0, p1);
        if (prev) store_out2<OT>(s.out, i, p0, p1);
        if constexpr (ALGO == ALGO_ADAMW) {
            adamw_pair_fused(p0, p1, g0, g1, m0, m1, v0, v1, c);   // adamw<true> on each, short roots
        } else {
            p0 = lion(p0, g0, m0, c);
            p1 = lion(p1, g1, m1, c);
        }
        store_master2<PT, SR>(s, i, p0, p1, idx);
        store_moment2<MV, SR>(s.m, i, m0, m1, idx, s.seed_m);
        if constexpr (ALGO == ALGO_ADAMW) store_moment2<MV, SR>(s.v, i, v0, v1, idx, s.seed_v);
        if (!prev) store_out2<OT>(s.out, i, p0, p1);
    }
    // the rest one element per lane: misaligned buffers, a ragged end, the scalar tail
    for (int64_t i = vend + threadIdx.x; i < hi; i += kThreads) {
        const uint32_t idx = s.idx0 + (uint32_t)i;
        const float g = load1<GT>(s.g, i);
        float m = load1<MV>(s.m, i);
        float p = load_master1<PT>(s, i);
        if (prev) store_out1<OT>(s.out, i, p);
        if constexpr (ALGO == ALGO_ADAMW) {
            float v = load1<MV>(s.v, i);
            p = adamw_sel(p, g, m, v, c, i < n_main);
            store_moment1<MV, SR>(s.v, i, v, SR ? hash32(idx ^ s.seed_v) : 0u);
        } else {
            p = lion(p, g, m, c);
        }
        p = store_master1<PT, SR>(s, i, p, idx);
        store_moment1<MV, SR>(s.m, i, m, SR ? hash32(idx ^ s.seed_m) : 0u);
        if (!prev) store_out1<OT>(s.out, i, p);
    }
}

template <int ALGO, int MV, int PT, int GT, int OT>
__global__ __launch_bounds__(kThreads) void k_update(Launch L)
{
    const int64_t tile = block_tile(L);
    if (tile >= L.ntiles) return;
    const DevSeg s = find_segment(L, tile);
    if (s.flags & kSR) update_tile<ALGO, MV, PT, GT, OT, true>(s, tile, L.tile);
    else update_tile<ALGO, MV, PT, GT, OT, false>(s, tile, L.tile);
}

// ------------------------------------------------------------ FP8 moment kernel

// 8 FP8 codes through byte accesses (buffers without 8-byte alignment).
__device__ __forceinline__ u32x2 load_codes8(const uint8_t* q)
{
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int k = 0; k < 8; ++k) w[k >> 2] |= (uint32_t)ld(q + k) << (8 * (k & 3));
    return u32x2{w[0], w[1]};
}

__device__ __forceinline__ void store_codes8(uint8_t* q, const uint32_t (&w)[2])
{
#pragma unroll
    for (int k = 0; k < 8; ++k) st(q + k, (uint8_t)(w[k >> 2] >> (8 * (k & 3))));
}

// The 8 codes of a lane (two words, byte k & 3 of word k >> 2) as FP32: packed conversions, and
// on a lane holding a NaN code, per-code conversions that keep the NaN's sign.
template <bool E5M2>
__device__ __forceinline__ void decode_codes(const u32x2 w, float (&x)[8])
{
    fp8_decode2<E5M2, false>(w.x, x[0], x[1]);
    fp8_decode2<E5M2, true>(w.x, x[2], x[3]);
    fp8_decode2<E5M2, false>(w.y, x[4], x[5]);
    fp8_decode2<E5M2, true>(w.y, x[6], x[7]);
    // the packed conversions give NaN exactly for NaN codes: one unordered compare per pair
    if (!(__builtin_isunordered(x[0], x[1]) | __builtin_isunordered(x[2], x[3]) |
          __builtin_isunordered(x[4], x[5]) | __builtin_isunordered(x[6], x[7])))
        return;
    if constexpr (E5M2) {
        x[0] = e5m2_decode<0>(w.x); x[1] = e5m2_decode<1>(w.x); x[2] = e5m2_decode<2>(w.x); x[3] = e5m2_decode<3>(w.x);
        x[4] = e5m2_decode<0>(w.y); x[5] = e5m2_decode<1>(w.y); x[6] = e5m2_decode<2>(w.y); x[7] = e5m2_decode<3>(w.y);
    } else {
        x[0] = e4m3_decode<0>(w.x); x[1] = e4m3_decode<1>(w.x); x[2] = e4m3_decode<2>(w.x); x[3] = e4m3_decode<3>(w.x);
        x[4] = e4m3_decode<0>(w.y); x[5] = e4m3_decode<1>(w.y); x[6] = e4m3_decode<2>(w.y); x[7] = e4m3_decode<3>(w.y);
    }
}

// x[k] / scale in place for a lane's 8 elements of one block (see block_div).  PLAIN: no value is
// -0 or NaN (block_quot_fast).
template <bool PLAIN>
__device__ __forceinline__ void block_quotients(float (&x)[8], const BlockDiv& d)
{
    if (d.fast && d.pre == 1.0f) {
#pragma unroll
        for (int k = 0; k < 8; ++k) x[k] = block_quot_fast<false, PLAIN>(x[k], d);
    } else if (d.fast) {
#pragma unroll
        for (int k = 0; k < 8; ++k) x[k] = block_quot_fast<true, PLAIN>(x[k], d);
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) x[k] = x[k] / d.s;
    }
}

// One DPP move: lane i reads lane perm(i) of its own row of 16 (the whole row is active).
template <int CTRL>
__device__ __forceinline__ uint32_t row_dpp(uint32_t u)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, CTRL, 0xf, 0xf, false);
}

// Max over the 16 lanes of a block group, which form one DPP row of the wavefront (lanes
// 16r .. 16r + 15).  The values are >= 0 and never NaN, so they order as their bits: four
// unsigned maxima, each with another lane's value -- within pairs, within quads (quad_perm
// [1,0,3,2] and [2,3,0,1]), then across half rows (row_half_mirror, lane i <-> 7 - i) and halves
// (row_mirror, lane i <-> 15 - i).
__device__ __forceinline__ float group16_max(float x)
{
    uint32_t u = fbits(x);
    u = __builtin_elementwise_max(u, row_dpp<0xb1>(u));
    u = __builtin_elementwise_max(u, row_dpp<0x4e>(u));
    u = __builtin_elementwise_max(u, row_dpp<0x141>(u));
    u = __builtin_elementwise_max(u, row_dpp<0x140>(u));
    return bitsf(u);
}

// Whether every one of a lane's 8 values lies in the range where gfx950's conversion instructions
// give fp8_encode's code (fp8_hw_range): one unsigned maximum of their offsets, no branches.
template <bool E5M2, bool SR>
__device__ __forceinline__ bool hw_range8(const float (&x)[8])
{
    uint32_t worst = 0u;
#pragma unroll
    for (int k = 0; k < 8; ++k) worst = __builtin_elementwise_max(worst, fp8_hw_offset<E5M2, SR>(x[k]));
    return worst <= fp8_hw_span<E5M2, SR>;
}

// A lane's 8 codes (two words, byte k & 3 of word k >> 2) through gfx950's conversion
// instructions; they are the reference's codes where hw_range8 holds (otherwise the words are to
// be recomputed in software).  idx % 8 == 0: FP8 segments start at multiples of 128 elements and
// a lane's group at a multiple of 8, so the 8 rounding streams share one hash head.
template <bool E5M2, bool SR>
__device__ __forceinline__ void hw_codes8(const float (&x)[8], uint32_t idx, uint32_t seed, const Wave8& w,
                                          uint32_t (&q)[2])
{
    if constexpr (SR) {
        uint32_t r[8];
        hash8(idx, seed, w, r);
        uint32_t w = fp8_hw_sr<E5M2, 0>(x[0], r[0], 0u);
        w = fp8_hw_sr<E5M2, 1>(x[1], r[1], w);
        w = fp8_hw_sr<E5M2, 2>(x[2], r[2], w);
        q[0] = fp8_hw_sr<E5M2, 3>(x[3], r[3], w);
        w = fp8_hw_sr<E5M2, 0>(x[4], r[4], 0u);
        w = fp8_hw_sr<E5M2, 1>(x[5], r[5], w);
        w = fp8_hw_sr<E5M2, 2>(x[6], r[6], w);
        q[1] = fp8_hw_sr<E5M2, 3>(x[7], r[7], w);
    } else {
        q[0] = fp8_hw_rne2<E5M2, true>(x[2], x[3], fp8_hw_rne2<E5M2, false>(x[0], x[1], 0u));
        q[1] = fp8_hw_rne2<E5M2, true>(x[6], x[7], fp8_hw_rne2<E5M2, false>(x[4], x[5], 0u));
    }
}

// FP8 block scale: absmax / format max, 1 for an all-zero block (kernels.c:1049-1057), correctly
// rounded.  The division by the constant multiplies by its correctly rounded reciprocal and
// applies one residual correction, which yields the correctly rounded quotient for every absmax
// >= 2^-100 (checked exhaustively over all floats, for both 448 and 57344); smaller ones divide.
template <bool E5M2>
__device__ __forceinline__ float block_scale(float amax)
{
    constexpr float kMax = E5M2 ? 57344.0f : 448.0f;
    constexpr float kInv = E5M2 ? 0x1.24924ap-16f : 0x1.24924ap-9f;   // RN(1 / kMax)
    if (!(amax > 0.0f)) return 1.0f;
    if (amax < 0x1p-100f) return amax / kMax;
    const float q = amax * kInv;
    const float r = __builtin_fmaf(-q, kMax, amax);
    return (r < 0.0f || r > 0.0f) ? __builtin_fmaf(r, kInv, q) : q;   // r zero or NaN (inf): q
}

// One 128-element block, 16 lanes x 8 elements (this lane: e0 .. e0 + 7): decode both moments,
// update, store master and output, block maxima by DPP within the 16 lanes, scales, codes.
// FULL: the whole block lies inside the segment, takes the fused form and allows vector access --
// straight-line code.  FULL is the same for the 16 lanes of a block, so the DPP maxima below always
// run with the whole group active.  base: the workgroup's first element of this pass over its tile
// (uniform, a multiple of the FP8 quantum); off = 8 x the lane's index in the workgroup, so the
// lane's elements start at e0 = base + off and its block at base + (off & ~127).  Vector accesses
// address base's byte offset (scalar) plus the lane's (lane_ptr).
template <int ALGO, int PT, int GT, int OT, bool SR, bool FULL, bool PREV>
__device__ __forceinline__ void fp8_block(const DevSeg& s, const Coef& c, int64_t base, uint32_t off)
{
    constexpr bool kLion = ALGO == ALGO_LION;
    constexpr int kGB = GT == DT_BF16 ? 2 : 4, kOB = OT == DT_BF16 ? 2 : 4, kPB = PT == DT_F24 ? 2 : 4;
    // block records: AdamW with an FP32 master (DT_PACKED8) or an FP24 master (DT_PACKED8_F24), Lion
    // with an FP32 master (DT_PACKED8_LION: the m codes in element order at 512) or an FP24 master
    // (DT_PACKED8_LION_F24: at 384)
    constexpr bool kRecF24 = PT == DT_PACKED8_F24 || PT == DT_PACKED8_LION_F24;
    constexpr bool kRecLion = PT == DT_PACKED8_LION || PT == DT_PACKED8_LION_F24;
    constexpr bool kRec = PT == DT_PACKED8 || kRecF24 || kRecLion;
    constexpr uint32_t kRecB = PT == DT_PACKED8 ? (uint32_t)kRecordBytes
                             : PT == DT_PACKED8_LION ? (uint32_t)kRecordBytesLion8
                             : PT == DT_PACKED8_LION_F24 ? (uint32_t)kRecordBytesLion8F24 : (uint32_t)kRecordBytesF24;
    constexpr uint32_t kCodesAt = PT == DT_PACKED8 ? 512u : 384u;   // the AdamW records' code slots
    constexpr uint32_t kLoAt = PT == DT_PACKED8_LION ? 512u : 256u; // the 8-byte slots: low bytes, Lion codes
    constexpr uint32_t kLionCodes = PT == DT_PACKED8_LION_F24 ? 128u : 0u;   // Lion's codes past rec_lo
    constexpr int kMaster = kRecF24 ? DT_F24 : kRecLion ? DT_PACKED8 : PT;   // how the 8 masters are coded
    const int64_t n = s.n, n_main = s.n_main;
    const bool vec = FULL || (s.flags & kVec) != 0;
    uint8_t* const mq = static_cast<uint8_t*>(s.m);
    uint8_t* const vq = static_cast<uint8_t*>(s.v);
    const int64_t e0 = base + off;
    const uint32_t idx = s.idx0 + (uint32_t)e0;
    const Wave8 w8 = SR ? wave8_of(idx) : Wave8{1u, 0u};   // for hash8
    const bool full = FULL || (vec && e0 + 8 <= n);
    const uint32_t lane = (off >> 3) & 15u;         // within the block's 16
    const uint32_t blk = off >> 7;                   // the block within this pass
    const int64_t ublk = base / kFp8Block;           // the pass's first block
    // records: the lane's 16-byte slot in its block's record (FP24 master high halves, or the
    // first half of an FP32 master with the second 256 bytes on; AdamW's codes kCodesAt bytes on) and
    // its 8-byte slot (FP24 low bytes; Lion's codes).  Computed once: the stores take them again
    // through fresh(), which keeps their scalar-base form without recomputing them.
    const uint32_t rec_lane = blk * kRecB + lane * 16u;
    const uint32_t rec_lo = blk * kRecB + kLoAt + lane * 8u;
    // Block scales: ordinary (cached) accesses.  A wavefront reads and writes 16 bytes of each
    // scale array, four blocks' worth; through L2 the four wavefronts of a workgroup share whole
    // lines, where non-temporal accesses sent each 16-byte piece to HBM on its own (measured: the
    // launch 3-4% slower, reads and writes 1.4% above the algorithmic bytes).
    const float sm = *(const ABH_GLOBAL float*)lane_ptr<float>(s.m_scale, ublk * 4, blk * 4u);
    const float sv = kLion ? 0.0f : *(const ABH_GLOBAL float*)lane_ptr<float>(s.v_scale, ublk * 4, blk * 4u);
    // the master's (pm, pl) and the output's (po) vector addresses for the lane offset o and, in
    // records, the lane's slots ro (rec_lane) and rl (rec_lo)
    auto pm = [&](uint32_t o, uint32_t ro) -> void* {
        if constexpr (kRec) return lane_ptr<void>(s.p, ublk * kRecB, ro);
        else return lane_ptr<void>(s.p, base * kPB, o * (uint32_t)kPB);
    };
    auto pl = [&](uint32_t o, uint32_t rl) -> uint8_t* {
        if constexpr (PT == DT_F24) return lane_ptr<uint8_t>(s.p_lo, base, o);
        else if constexpr (kRecF24) return lane_ptr<uint8_t>(s.p, ublk * kRecB, rl);
        else return nullptr;
    };
    auto po = [&](uint32_t o) -> void* {
        if constexpr (OT != DT_NONE) return lane_ptr<void>(s.out, base * kOB, o * (uint32_t)kOB);
        else return nullptr;
    };
    // codes are stored padded to whole blocks, so all 8 of this lane's exist
    u32x2 cm, cv = {0u, 0u};
    if constexpr (kRecLion) {
        cm = ld(lane_ptr<const u32x2>(s.p, ublk * kRecB, rec_lo + kLionCodes));
    } else if constexpr (kRec) {
        const u32x4 w = ld(lane_ptr<const u32x4>(s.p, ublk * kRecB, rec_lane + kCodesAt));
        cm = u32x2{w.x, w.y};
        cv = u32x2{w.z, w.w};
    } else {
        cm = vec ? ld(lane_ptr<const u32x2>(mq, base, off)) : load_codes8(mq + e0);
        if constexpr (!kLion) cv = vec ? ld(lane_ptr<const u32x2>(vq, base, off)) : load_codes8(vq + e0);
    }
    // Full blocks of records load their masters only once the moments' quotients are computed
    // (kDefer): the lane's first requests (codes, gradients) go out alone and the masters' after
    // them, fewer bytes in flight at once (the 7B list in interleaved A/B runs: FP24 masters 16.32
    // against 16.40 ms, FP32 masters 18.36 against 18.52).
    constexpr bool kDefer = kRec && FULL && !kLion && !PREV;
    float g[8], p[8], mt[8], vt[8];
    if (full) {
        load8<GT>(lane_ptr<const void>(s.g, base * kGB, off * (uint32_t)kGB), g);
        if constexpr (!kDefer) load_master8<kMaster>(pm(off, rec_lane), pl(off, rec_lo), p);
        if constexpr (PREV) store_out8<OT>(po(off), p);   // out from the master as loaded
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const bool in = e0 + k < n;
            g[k] = in ? load1<GT>(s.g, e0 + k) : 0.0f;
            p[k] = in ? load_master1<PT>(s, e0 + k) : 0.0f;
            if (PREV && in) store_out1<OT>(s.out, e0 + k, p[k]);
        }
    }
    {
        float d[8];
        decode_codes<false>(cm, d);
#pragma unroll
        for (int k = 0; k < 8; ++k) mt[k] = d[k] * sm;
        if constexpr (!kLion) {
            decode_codes<true>(cv, d);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float u = d[k] * sv;
                vt[k] = u * u;
            }
        }
    }
    // the update, FP32 moments in registers; sq = sqrt(new v), reused for the v code below
    float sq[8];
    const bool lane_fused = FULL || kLion || e0 + 8 <= n_main;
    bool v_pos = false;     // every new v of the wavefront positive and finite (uniform)
    bool m_plain = false;   // every new m of the wavefront finite, 2^-60 <= |m| <= 2^60 (uniform)
    float m_low = 0.0f;     // where m_plain: the lane's smallest |m|
    if constexpr (kDefer) {
        float q[8];
        v_pos = adamw8_fused_q(g, mt, vt, c, sq, (s.flags & kFastDiv) != 0, m_plain, m_low, q);
        uint32_t ro = rec_lane, rl = rec_lo;   // offsets that depend on q: the loads cannot move up
        asm volatile("" : "+v"(ro), "+v"(rl) : "v"(q[0]));
        load_master8<kMaster>(pm(off, ro), pl(off, rl), p);
#pragma unroll
        for (int k = 0; k < 8; ++k) p[k] = __builtin_fmaf(-c.step, q[k], p[k] * c.decay);
    } else if constexpr (FULL && !kLion) {
        v_pos = adamw8_fused(p, g, mt, vt, c, sq, (s.flags & kFastDiv) != 0, m_plain, m_low);
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if constexpr (kLion) p[k] = lion(p[k], g[k], mt[k], c);
            else p[k] = lane_fused ? adamw<true>(p[k], g[k], mt[k], vt[k], c, sq[k])
                                   : adamw_sel(p[k], g[k], mt[k], vt[k], c, e0 + k < n_main, sq[k]);
        }
    }
    if (full) {
        const uint32_t o = fresh(off);
        const uint32_t ro = kRec ? fresh(rec_lane) : 0u, rl = kRecF24 ? fresh(rec_lo) : 0u;
        store_master8<kMaster, SR>(pm(o, ro), pl(o, rl), p, idx, s.seed_p, w8);
        if constexpr (!PREV) store_out8<OT>(po(o), p);
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if (e0 + k < n) {
                const float stored = store_master1<PT, SR>(s, e0 + k, p[k], idx + k);
                if (!PREV) store_out1<OT>(s.out, e0 + k, stored);
            }
        }
    }
    // block maxima (NaN skipped), elements past the end count as zero.  v is stored as
    // u = sqrt(max(v, 0)) (kernels.c:893-905).  The new v is never -0 (an FMA of a product and a
    // sum of exact zeros rounds to +0), so u is sq (the same correctly rounded root) wherever sq is
    // not NaN, i.e. v >= 0, and 0 where it is (v < 0 or NaN).  Where v_pos holds, u = sq throughout,
    // and the lane's smallest u serves the conversion instructions' range test below.  Otherwise sq
    // keeps its NaNs (read here, not rewritten: a rewrite would have the branches hand sq over in
    // different registers), v_nan marks them, and the integer encoder below codes 0 there.
    float am = 0.0f, au = 0.0f, u_min = 0.0f;
    uint32_t v_nan = 0u;   // bit k: sq[k] is NaN
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        if (!FULL && e0 + k >= n) { mt[k] = 0.0f; sq[k] = 0.0f; }
        am = __builtin_fmaxf(am, fabsf(mt[k]));   // a NaN m is skipped (IEEE maxNum)
    }
    if constexpr (!kLion) {
        if (v_pos) {   // positive floats order as their bits
            uint32_t ub = 0u, lb = 0xffffffffu;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                ub = __builtin_elementwise_max(ub, fbits(sq[k]));
                lb = __builtin_elementwise_min(lb, fbits(sq[k]));
            }
            au = bitsf(ub);
            u_min = bitsf(lb);
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                au = sq[k] > au ? sq[k] : au;   // a NaN is skipped
                v_nan |= sq[k] != sq[k] ? 1u << k : 0u;
            }
        }
    }
    am = group16_max(am);
    const float scm = block_scale<false>(am);
    float scu = 1.0f;
    if constexpr (!kLion) {
        au = group16_max(au);
        scu = block_scale<true>(au);
    }
    {
        const BlockDiv dm = block_div(scm, am);
        if (m_plain) block_quotients<true>(mt, dm);
        else block_quotients<false>(mt, dm);
    }
    if constexpr (!kLion) block_quotients<true>(sq, block_div(scu, au));
    // codes: full blocks through the conversion instructions; a lane holding a value outside
    // their exact range (rare: zeros, values below the smallest normal after scaling, NaN) and
    // partial blocks take the integer encoder.  Where m_plain (v_pos) holds, the lane's values
    // are finite and nonzero, and each quotient reaches the smallest normal 2^-6 (2^-14) once the
    // smallest |m| (u) reaches that multiple of the scale (rounding is monotone, and the multiple is
    // exact: |m| >= 2^-60 and u >= 2^-50 there keep the scales above 2^-69 and 2^-66); the per-value
    // test is needed otherwise.
    uint32_t qm[2] = {0u, 0u}, qv[2] = {0u, 0u};
    bool soft_m = true, soft_v = !kLion;
    if constexpr (FULL) {
        hw_codes8<false, SR>(mt, idx, s.seed_m, w8, qm);
        soft_m = !(m_plain ? (!SR || m_low >= scm * 0x1p-6f) : hw_range8<false, SR>(mt));
        if constexpr (!kLion) {
            hw_codes8<true, SR>(sq, idx, s.seed_v, w8, qv);
            soft_v = !(v_pos ? (!SR || u_min >= scu * 0x1p-14f) : hw_range8<true, SR>(sq));
        }
    }
    if (soft_m) {
        qm[0] = qm[1] = 0u;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const bool in = FULL || e0 + k < n;   // padding codes are zero
            const uint32_t a = e4m3_encode<SR>(mt[k], SR ? hash32((idx + k) ^ s.seed_m) : 0u);
            qm[k >> 2] |= (in ? a : 0u) << (8 * (k & 3));
        }
    }
    if (soft_v) {
        qv[0] = qv[1] = 0u;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const bool in = FULL || e0 + k < n;
            const float u = (v_nan >> k) & 1u ? 0.0f : sq[k];   // u / scale: 0 where sq was NaN
            const uint32_t b = e5m2_encode<SR>(u, SR ? hash32((idx + k) ^ s.seed_v) : 0u);
            qv[k >> 2] |= (in ? b : 0u) << (8 * (k & 3));
        }
    }
    const uint32_t o = fresh(off);
    if constexpr (kRecLion) {
        st(lane_ptr<u32x2>(s.p, ublk * kRecB, fresh(rec_lo) + kLionCodes), u32x2{qm[0], qm[1]});
    } else if constexpr (kRec) {
        st(lane_ptr<u32x4>(s.p, ublk * kRecB, fresh(rec_lane) + kCodesAt), u32x4{qm[0], qm[1], qv[0], qv[1]});
    } else if (vec) {
        st(lane_ptr<u32x2>(mq, base, o), u32x2{qm[0], qm[1]});
        if constexpr (!kLion) st(lane_ptr<u32x2>(vq, base, o), u32x2{qv[0], qv[1]});
    } else {
        store_codes8(mq + e0, qm);
        if constexpr (!kLion) store_codes8(vq + e0, qv);
    }
    if (lane == 0) {
        *(ABH_GLOBAL float*)lane_ptr<float>(s.m_scale, ublk * 4, (o >> 7) * 4u) = scm;
        if constexpr (!kLion) *(ABH_GLOBAL float*)lane_ptr<float>(s.v_scale, ublk * 4, (o >> 7) * 4u) = scu;
    }
}

template <int ALGO, int PT, int GT, int OT, bool SR, bool PREV, bool WIDE>
__device__ __forceinline__ void update_tile_fp8(const DevSeg& s, int64_t tile, int64_t T)
{
    constexpr bool kLion = ALGO == ALGO_LION;
    const Coef c = s.c;
    const uint32_t off = threadIdx.x * 8u;   // 16-lane group g holds block g of each pass
    const int64_t goff = (int64_t)(off & ~(uint32_t)(kFp8Block - 1));
    const bool vec = (s.flags & kVec) != 0;
    // blocks wholly in the fused range (AdamW's scalar tail, if any, is the segment's last n mod W)
    const int64_t full_end = kLion ? s.n : s.n_main;
    if constexpr (!WIDE) {
        // The smallest tile (the default) holds one 128-element block per 16-lane group: no loop and
        // no loop-carried addresses (measured 1.3% faster on the 7B FP8 step in a fast HBM placement,
        // equal in a slow one)
        const int64_t base = (tile - s.tile_begin) * kFp8Quantum;
        const int64_t b0 = base + goff;
        if (b0 >= s.n) return;
        if (vec && b0 + kFp8Block <= full_end) fp8_block<ALGO, PT, GT, OT, SR, true, PREV>(s, c, base, off);
        else fp8_block<ALGO, PT, GT, OT, SR, false, PREV>(s, c, base, off);
    } else {
        const int64_t lo = (tile - s.tile_begin) * T;
        const int64_t hi = lo + T < s.n ? lo + T : s.n;
        // larger tiles (ADAMBRIDGE_TILE_FP8): each pass covers the next 16 blocks of the tile
        for (int64_t base = lo; base + goff < hi; base += kFp8Quantum) {
            const int64_t b0 = base + goff;
            if (vec && b0 + kFp8Block <= full_end) fp8_block<ALGO, PT, GT, OT, SR, true, PREV>(s, c, base, off);
            else fp8_block<ALGO, PT, GT, OT, SR, false, PREV>(s, c, base, off);
        }
    }
}

// WIDE: the launch's tiles hold more than one block per 16-lane group (ADAMBRIDGE_TILE_FP8 above
// 2048).  The default tile takes the kernel without the loop: 58 VGPRs for the FP8-record and FP24
// variants, room for 8 wavefronts per SIMD, where the loop in the same kernel made it 89-102 (5).
// The FP24-master forms use all 8: the 7B list with an FP24 master took 16.52 ms per launch
// against 18.5-19.0 at 5.  (launch_lds holds the FP32-master AdamW forms at 6 workgroups per CU.)
// A pipelined form of the loop for block records, each pass's loads issued during the previous
// pass's arithmetic, took 111-113 VGPRs (4 wavefronts per SIMD) and was 7-13% slower at 4096-16384
// element tiles than this form at 2048.
template <int ALGO, int PT, int GT, int OT, bool WIDE>
__global__ __launch_bounds__(kThreads) void k_update_fp8(Launch L)
{
    const int64_t tile = block_tile(L);
    if (tile >= L.ntiles) return;
    const DevSeg s = find_segment(L, tile);
    // the out-from-previous-master form is its own instantiation: a runtime test inside the block
    // code cost this VALU-heavy kernel 6% (measured on the 7B FP8 step)
    if (s.flags & kPrev) {
        if constexpr (OT != DT_NONE) {
            if (s.flags & kSR) update_tile_fp8<ALGO, PT, GT, OT, true, true, WIDE>(s, tile, L.tile);
            else update_tile_fp8<ALGO, PT, GT, OT, false, true, WIDE>(s, tile, L.tile);
        }
        return;
    }
    if (s.flags & kSR) update_tile_fp8<ALGO, PT, GT, OT, true, false, WIDE>(s, tile, L.tile);
    else update_tile_fp8<ALGO, PT, GT, OT, false, false, WIDE>(s, tile, L.tile);
}

// ------------------------------------------------- packed AdamW state kernel
//
// AdamW with an FP32 master and BF16 moments interleaved in HBM: for elements
// 2k and 2k+1 of a segment, 16 bytes {p[2k], p[2k+1], m[2k] | m[2k+1] << 16,
// v[2k] | v[2k+1] << 16}.  One 16-byte state access per lane instead of three
// separate streams (master, m, v): fewer concurrent DRAM streams, measured
// faster on MI355X.  s.p holds the state; s.p_lo the buffer that receives the
// new state (the same pointer, or a second buffer when double-buffered).  The
// arithmetic and rounding are those of the separate layout, element by element.

__device__ __forceinline__ void adamw_pair_tail(const DevSeg& s, int64_t i, u32x4& x, float g0, float g1,
                                                int nvalid, uint32_t idx, bool sr, int64_t n_main,
                                                float& o0, float& o1)
{
    // slow path for a pair that holds a tail element or ends past n: element by element
    float p[2] = {bitsf(x.x), bitsf(x.y)};
    float m[2] = {bitsf(x.z << 16), bitsf(x.z & 0xffff0000u)};
    float v[2] = {bitsf(x.w << 16), bitsf(x.w & 0xffff0000u)};
    const float g[2] = {g0, g1};
    uint32_t mh[2] = {x.z & 0xffffu, x.z >> 16}, vh[2] = {x.w & 0xffffu, x.w >> 16};
    uint32_t pb[2] = {x.x, x.y};
    for (int k = 0; k < nvalid; ++k) {
        p[k] = adamw_sel(p[k], g[k], m[k], v[k], s.c, i + k < n_main);
        pb[k] = fbits(p[k]);
        mh[k] = sr ? bf16_store<true>(m[k], hash32((idx + k) ^ s.seed_m)) : bf16_store<false>(m[k], 0u);
        vh[k] = sr ? bf16_store<true>(v[k], hash32((idx + k) ^ s.seed_v)) : bf16_store<false>(v[k], 0u);
    }
    x = u32x4{pb[0], pb[1], mh[0] | (mh[1] << 16), vh[0] | (vh[1] << 16)};
    o0 = p[0];
    o1 = p[1];
}

// The working weights of elements i and (if both) i + 1.
template <int OT>
__device__ __forceinline__ void store_pair_out(void* out, int64_t i, bool vec2, bool both, float o0, float o1)
{
    if (vec2) store_out2<OT>(out, i, o0, o1);
    else {
        store_out1<OT>(out, i, o0);
        if (both) store_out1<OT>(out, i + 1, o1);
    }
}

template <int GT, int OT, bool SR>
__device__ __forceinline__ void update_tile_packed(const DevSeg& s, int64_t tile, int64_t T)
{
    const int64_t n = s.n, n_main = s.n_main;
    const Coef c = s.c;
    const u32x4* __restrict__ src = static_cast<const u32x4*>(s.p);
    u32x4* __restrict__ dst = reinterpret_cast<u32x4*>(s.p_lo);
    const bool vec = (s.flags & kVec) != 0;   // g and out allow 2-element access
    const bool prev = (s.flags & kPrev) != 0;  // uniform: out from the master as loaded
    const int64_t lo = (tile - s.tile_begin) * T;
    const int64_t hi = lo + T < n ? lo + T : n;
    for (int64_t i = lo + threadIdx.x * 2; i < hi; i += kThreads * 2) {
        const int64_t pair = i >> 1;
        const uint32_t idx = s.idx0 + (uint32_t)i;
        u32x4 x = ld(src + pair);
        const bool both = i + 2 <= n;
        float g0 = 0.0f, g1 = 0.0f;
        if (vec && both) load2<GT>(s.g, i, g0, g1);
        else {
            g0 = load1<GT>(s.g, i);
            if (both) g1 = load1<GT>(s.g, i + 1);
        }
        if (prev) store_pair_out<OT>(s.out, i, vec && both, both, bitsf(x.x), bitsf(x.y));
        float o0, o1;
        if (i + 2 <= n_main) {
            float p0 = bitsf(x.x), p1 = bitsf(x.y);
            float m0 = bitsf(x.z << 16), m1 = bitsf(x.z & 0xffff0000u);
            float v0 = bitsf(x.w << 16), v1 = bitsf(x.w & 0xffff0000u);
            adamw_pair_fused(p0, p1, g0, g1, m0, m1, v0, v1, c);
            const uint32_t mw = bf16_store<SR>(m0, SR ? hash32(idx ^ s.seed_m) : 0u) |
                                (bf16_store<SR>(m1, SR ? hash32((idx + 1) ^ s.seed_m) : 0u) << 16);
            const uint32_t vw = bf16_store<SR>(v0, SR ? hash32(idx ^ s.seed_v) : 0u) |
                                (bf16_store<SR>(v1, SR ? hash32((idx + 1) ^ s.seed_v) : 0u) << 16);
            x = u32x4{fbits(p0), fbits(p1), mw, vw};
            o0 = p0;
            o1 = p1;
        } else {
            adamw_pair_tail(s, i, x, g0, g1, both ? 2 : 1, idx, SR, n_main, o0, o1);
        }
        st(dst + pair, x);
        if (!prev) store_pair_out<OT>(s.out, i, vec && both, both, o0, o1);
    }
}

template <int GT, int OT>
__global__ __launch_bounds__(kThreads) void k_update_packed(Launch L)
{
    const int64_t tile = block_tile(L);
    if (tile >= L.ntiles) return;
    const DevSeg s = find_segment(L, tile);
    if (s.flags & kSR) update_tile_packed<GT, OT, true>(s, tile, L.tile);
    else update_tile_packed<GT, OT, false>(s, tile, L.tile);
}

// ------------------------------------------------------ Lion record state kernel
//
// Lion with an FP32 master and a BF16 moment in one 1536-byte record per 256
// elements: the record's 256 masters in element order, then its 256 m values
// (BF16 bits) in element order.  Each lane takes 4 consecutive elements, so a
// wavefront covers one record per pass: one 16-byte master access and one
// 8-byte moment access per lane, each instruction over one contiguous span
// (1024 and 512 bytes), and 8-byte gradient and output accesses.  Measured on
// MI355X over the Qwen2.5-1.5B parameter list (1.54G elements): 3.95 ms per
// step against 4.03-4.08 ms in the separate layout, 4.08 ms in 768-byte records
// of 128 elements (2 per lane) and 4.26 ms in 3072-byte records of 512 (8 per
// lane), all timed in turn in one process.  Lion fuses every element
// (kernels.c:1093-1106), so there is no scalar tail; a record's slots past n
// are padding and are written back unchanged.
//
// With an FP32 moment (MV = DT_F32, ADAMBRIDGE_DT_PACKED_LION_F32): 2048-byte records, the 256
// masters and then the 256 m values, both FP32 and stored exactly -- a 16-byte moment access per
// lane, the FP32-moment AdamW records' access shape.

constexpr int64_t kLionRecordElems = 256;
constexpr int64_t kLionRecordBytes = 1536;
constexpr int64_t kLionF32RecordBytes = 2048;

// The working weights of elements i .. i + 3 below n, from FP32 bits.
template <int OT>
__device__ __forceinline__ void store_quad_out(void* out, int64_t i, int64_t n, bool vec4, const uint32_t (&p)[4])
{
    if (vec4) {
        store_out2<OT>(out, i, bitsf(p[0]), bitsf(p[1]));
        store_out2<OT>(out, i + 2, bitsf(p[2]), bitsf(p[3]));
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (i + k < n) store_out1<OT>(out, i + k, bitsf(p[k]));
    }
}

template <int GT, int OT, bool SR, int MV>
__device__ __forceinline__ void update_tile_lion_rec(const DevSeg& s, int64_t tile, int64_t T)
{
    constexpr bool kF32 = MV == DT_F32;
    constexpr int64_t kRecB = kF32 ? kLionF32RecordBytes : kLionRecordBytes;
    const int64_t n = s.n;
    const Coef c = s.c;
    const uint8_t* __restrict__ src = static_cast<const uint8_t*>(s.p);
    uint8_t* __restrict__ dst = s.p_lo;
    const bool vec = (s.flags & kVec) != 0;   // g and out allow 2-element access
    const bool prev = (s.flags & kPrev) != 0;  // uniform: out from the master as loaded
    const int64_t lo = (tile - s.tile_begin) * T;
    const int64_t hi = lo + T < n ? lo + T : n;
    for (int64_t i = lo + threadIdx.x * 4; i < hi; i += kThreads * 4) {
        // i % 4 == 0: record i / 256, masters at 4 (i % 256), m values at 1024 + 2 (i % 256) (BF16)
        // or 1024 + 4 (i % 256) (FP32)
        const int64_t rec = (i / kLionRecordElems) * kRecB;
        const int64_t at = rec + (i % kLionRecordElems) * 4;
        const int64_t at_m = rec + 1024 + (i % kLionRecordElems) * (kF32 ? 4 : 2);
        const uint32_t idx = s.idx0 + (uint32_t)i;
        const u32x4 pw = ld(reinterpret_cast<const u32x4*>(src + at));
        uint32_t m_in[4];
        if constexpr (kF32) {
            const u32x4 mw = ld(reinterpret_cast<const u32x4*>(src + at_m));
            m_in[0] = mw.x; m_in[1] = mw.y; m_in[2] = mw.z; m_in[3] = mw.w;
        } else {
            const u32x2 mw = ld(reinterpret_cast<const u32x2*>(src + at_m));
            m_in[0] = mw.x & 0xffffu; m_in[1] = mw.x >> 16; m_in[2] = mw.y & 0xffffu; m_in[3] = mw.y >> 16;
        }
        const bool all = i + 4 <= n;
        float g[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (vec && all) {
            load2<GT>(s.g, i, g[0], g[1]);
            load2<GT>(s.g, i + 2, g[2], g[3]);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (i + k < n) g[k] = load1<GT>(s.g, i + k);
        }
        const uint32_t p_in[4] = {pw.x, pw.y, pw.z, pw.w};
        if (prev) store_quad_out<OT>(s.out, i, n, vec && all, p_in);
        uint32_t p_out[4], m_out[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float m = bitsf(kF32 ? m_in[k] : m_in[k] << 16);
            const float p = lion(bitsf(p_in[k]), g[k], m, c);
            const bool in = all || i + k < n;   // padding keeps its bits
            p_out[k] = in ? fbits(p) : p_in[k];
            if constexpr (kF32) m_out[k] = in ? fbits(m) : m_in[k];
            else m_out[k] = in ? bf16_store<SR>(m, SR ? hash32((idx + k) ^ s.seed_m) : 0u) : m_in[k];
        }
        st(reinterpret_cast<u32x4*>(dst + at), u32x4{p_out[0], p_out[1], p_out[2], p_out[3]});
        if constexpr (kF32) st(reinterpret_cast<u32x4*>(dst + at_m), u32x4{m_out[0], m_out[1], m_out[2], m_out[3]});
        else st(reinterpret_cast<u32x2*>(dst + at_m), u32x2{m_out[0] | (m_out[1] << 16), m_out[2] | (m_out[3] << 16)});
        if (!prev) store_quad_out<OT>(s.out, i, n, vec && all, p_out);
    }
}

template <int GT, int OT>
__global__ __launch_bounds__(kThreads) void k_update_lion_rec(Launch L)
{
    const int64_t tile = block_tile(L);
    if (tile >= L.ntiles) return;
    const DevSeg s = find_segment(L, tile);
    if (s.flags & kSR) update_tile_lion_rec<GT, OT, true, DT_BF16>(s, tile, L.tile);
    else update_tile_lion_rec<GT, OT, false, DT_BF16>(s, tile, L.tile);
}

// The FP32 moment is stored exactly: no rounding stream, one form.
template <int GT, int OT>
__global__ __launch_bounds__(kThreads) void k_update_lion_f32rec(Launch L)
{
    const int64_t tile = block_tile(L);
    if (tile >= L.ntiles) return;
    const DevSeg s = find_segment(L, tile);
    update_tile_lion_rec<GT, OT, false, DT_F32>(s, tile, L.tile);
}

// --------------------------------------------- FP32-moment AdamW record kernel
//
// AdamW with an FP32 master and FP32 moments in one 3072-byte record per 256
// elements: the record's 256 masters, then its 256 m, then its 256 v, each
// in element order.  Each lane takes 4 consecutive elements: three 16-byte
// state accesses, each wavefront instruction one contiguous 1 KiB span, and
// 8-byte gradient and output accesses -- the access shape of the Lion records,
// in place of the separate layout's 8-byte accesses to three arrays.  Fused
// elements take the pair kernel's arithmetic (adamw_pair_fused); the scalar
// tail of the reproduced SIMD level the unfused form, element by element; a
// record's slots past n are padding and are written back unchanged.  FP32
// moments and master are stored exactly (no stochastic rounding).

constexpr int64_t kF32RecordElems = 256;
constexpr int64_t kF32RecordBytes = 3072;

template <int GT, int OT>
__device__ __forceinline__ void update_tile_f32rec(const DevSeg& s, int64_t tile, int64_t T)
{
    const int64_t n = s.n, n_main = s.n_main;
    const Coef c = s.c;
    const uint8_t* __restrict__ src = static_cast<const uint8_t*>(s.p);
    uint8_t* __restrict__ dst = s.p_lo;
    const bool vec = (s.flags & kVec) != 0;   // g and out allow 2-element access
    const bool prev = (s.flags & kPrev) != 0;  // uniform: out from the master as loaded
    const int64_t lo = (tile - s.tile_begin) * T;
    const int64_t hi = lo + T < n ? lo + T : n;
    for (int64_t i = lo + threadIdx.x * 4; i < hi; i += kThreads * 4) {
        // i % 4 == 0: record i / 256, masters at 4 (i % 256), m 1024 bytes on, v 2048 bytes on
        const int64_t at = (i / kF32RecordElems) * kF32RecordBytes + (i % kF32RecordElems) * 4;
        const u32x4 pw = ld(reinterpret_cast<const u32x4*>(src + at));
        const u32x4 mw = ld(reinterpret_cast<const u32x4*>(src + at + 1024));
        const u32x4 vw = ld(reinterpret_cast<const u32x4*>(src + at + 2048));
        const bool all = i + 4 <= n;
        float g[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (vec && all) {
            load2<GT>(s.g, i, g[0], g[1]);
            load2<GT>(s.g, i + 2, g[2], g[3]);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (i + k < n) g[k] = load1<GT>(s.g, i + k);
        }
        const uint32_t p_in[4] = {pw.x, pw.y, pw.z, pw.w};
        const uint32_t m_in[4] = {mw.x, mw.y, mw.z, mw.w};
        const uint32_t v_in[4] = {vw.x, vw.y, vw.z, vw.w};
        if (prev) store_quad_out<OT>(s.out, i, n, vec && all, p_in);
        float p[4], m[4], v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            p[k] = bitsf(p_in[k]);
            m[k] = bitsf(m_in[k]);
            v[k] = bitsf(v_in[k]);
        }
        if (i + 4 <= n_main) {
            adamw_pair_fused(p[0], p[1], g[0], g[1], m[0], m[1], v[0], v[1], c);
            adamw_pair_fused(p[2], p[3], g[2], g[3], m[2], m[3], v[2], v[3], c);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (i + k < n) p[k] = adamw_sel(p[k], g[k], m[k], v[k], c, i + k < n_main);
        }
        uint32_t p_out[4], m_out[4], v_out[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const bool in = all || i + k < n;   // padding keeps its bits
            p_out[k] = in ? fbits(p[k]) : p_in[k];
            m_out[k] = in ? fbits(m[k]) : m_in[k];
            v_out[k] = in ? fbits(v[k]) : v_in[k];
        }
        st(reinterpret_cast<u32x4*>(dst + at), u32x4{p_out[0], p_out[1], p_out[2], p_out[3]});
        st(reinterpret_cast<u32x4*>(dst + at + 1024), u32x4{m_out[0], m_out[1], m_out[2], m_out[3]});
        st(reinterpret_cast<u32x4*>(dst + at + 2048), u32x4{v_out[0], v_out[1], v_out[2], v_out[3]});
        if (!prev) store_quad_out<OT>(s.out, i, n, vec && all, p_out);
    }
}

template <int GT, int OT>
__global__ __launch_bounds__(kThreads) void k_update_f32rec(Launch L)
{
    const int64_t tile = block_tile(L);
    if (tile >= L.ntiles) return;
    const DevSeg s = find_segment(L, tile);
    update_tile_f32rec<GT, OT>(s, tile, L.tile);
}

// ------------------------------------------- FP24-master, BF16-moment AdamW record kernel
//
// AdamW with an FP24 master and BF16 moments in one 1792-byte record per 256
// elements: the record's 256 master high halves (BF16 bits), its 256 master low
// bytes, its 256 m and its 256 v (BF16 bits), each in element order.  4 elements
// a lane: 8-byte high-half, moment and gradient accesses and a 4-byte low-byte
// access, each wavefront instruction over one contiguous span of the record, in
// place of the separate layout's six arrays (two of them read 2 bytes a lane).
// Arithmetic as the FP32-moment records; the master is rounded to FP24 and the
// moments to BF16 with the separate layout's roundings and rounding streams.
//
// With FP32 moments (MV = DT_F32, ADAMBRIDGE_DT_PACKED_F24_F32): 2816-byte records, the same high
// halves and low bytes, then the 256 m and the 256 v as FP32 (16-byte accesses a lane), stored
// exactly.

constexpr int64_t kF24RecordElems = 256;
constexpr int64_t kF24RecordBytes = 1792;
constexpr int64_t kF24F32RecordBytes = 2816;

template <int GT, int OT, bool SR, int MV = DT_BF16>
__device__ __forceinline__ void update_tile_f24rec(const DevSeg& s, int64_t tile, int64_t T)
{
    constexpr bool kF32 = MV == DT_F32;
    constexpr int64_t kRecB = kF32 ? kF24F32RecordBytes : kF24RecordBytes;
    constexpr int64_t kMB = kF32 ? 4 : 2;   // bytes per moment value
    const int64_t n = s.n, n_main = s.n_main;
    const Coef c = s.c;
    const uint8_t* __restrict__ src = static_cast<const uint8_t*>(s.p);
    uint8_t* __restrict__ dst = s.p_lo;
    const bool vec = (s.flags & kVec) != 0;   // g and out allow 2-element access
    const bool prev = (s.flags & kPrev) != 0;  // uniform: out from the master as loaded
    const int64_t lo = (tile - s.tile_begin) * T;
    const int64_t hi = lo + T < n ? lo + T : n;
    for (int64_t i = lo + threadIdx.x * 4; i < hi; i += kThreads * 4) {
        // i % 4 == 0: record i / 256; high halves at 2j, low bytes at 512 + j, m at 768 + 2j and
        // v at 1280 + 2j (BF16), or m at 768 + 4j and v at 1792 + 4j (FP32), for j = i % 256
        const int64_t rec = (i / kF24RecordElems) * kRecB;
        const int64_t j = i % kF24RecordElems;
        const int64_t at_h = rec + 2 * j, at_l = rec + 512 + j, at_m = rec + 768 + kMB * j,
                      at_v = rec + 768 + 256 * kMB + kMB * j;
        const uint32_t idx = s.idx0 + (uint32_t)i;
        const u32x2 hw = ld(reinterpret_cast<const u32x2*>(src + at_h));
        const uint32_t lw = ld(reinterpret_cast<const uint32_t*>(src + at_l));
        uint32_t m_in[4], v_in[4];
        if constexpr (kF32) {
            const u32x4 mw = ld(reinterpret_cast<const u32x4*>(src + at_m));
            const u32x4 vw = ld(reinterpret_cast<const u32x4*>(src + at_v));
            m_in[0] = mw.x; m_in[1] = mw.y; m_in[2] = mw.z; m_in[3] = mw.w;
            v_in[0] = vw.x; v_in[1] = vw.y; v_in[2] = vw.z; v_in[3] = vw.w;
        } else {
            const u32x2 mw = ld(reinterpret_cast<const u32x2*>(src + at_m));
            const u32x2 vw = ld(reinterpret_cast<const u32x2*>(src + at_v));
            m_in[0] = mw.x & 0xffffu; m_in[1] = mw.x >> 16; m_in[2] = mw.y & 0xffffu; m_in[3] = mw.y >> 16;
            v_in[0] = vw.x & 0xffffu; v_in[1] = vw.x >> 16; v_in[2] = vw.y & 0xffffu; v_in[3] = vw.y >> 16;
        }
        const bool all = i + 4 <= n;
        float g[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (vec && all) {
            load2<GT>(s.g, i, g[0], g[1]);
            load2<GT>(s.g, i + 2, g[2], g[3]);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (i + k < n) g[k] = load1<GT>(s.g, i + k);
        }
        const uint32_t h_in[4] = {hw.x & 0xffffu, hw.x >> 16, hw.y & 0xffffu, hw.y >> 16};
        uint32_t p_in[4];   // the stored masters as FP32 bits: hi << 16 | lo << 8
#pragma unroll
        for (int k = 0; k < 4; ++k) p_in[k] = (h_in[k] << 16) | (((lw >> (8 * k)) & 0xffu) << 8);
        if (prev) store_quad_out<OT>(s.out, i, n, vec && all, p_in);
        float p[4], m[4], v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            p[k] = bitsf(p_in[k]);
            m[k] = bitsf(kF32 ? m_in[k] : m_in[k] << 16);
            v[k] = bitsf(kF32 ? v_in[k] : v_in[k] << 16);
        }
        if (i + 4 <= n_main) {
            adamw_pair_fused(p[0], p[1], g[0], g[1], m[0], m[1], v[0], v[1], c);
            adamw_pair_fused(p[2], p[3], g[2], g[3], m[2], m[3], v[2], v[3], c);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (i + k < n) p[k] = adamw_sel(p[k], g[k], m[k], v[k], c, i + k < n_main);
        }
        uint32_t p_out[4], m_out[4], v_out[4], l_out = 0u;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const bool in = all || i + k < n;   // padding keeps its bits
            p_out[k] = in ? f24_round<SR>(p[k], SR ? hash32((idx + k) ^ s.seed_p) : 0u) : p_in[k];
            if constexpr (kF32) {
                m_out[k] = in ? fbits(m[k]) : m_in[k];
                v_out[k] = in ? fbits(v[k]) : v_in[k];
            } else {
                m_out[k] = in ? bf16_store<SR>(m[k], SR ? hash32((idx + k) ^ s.seed_m) : 0u) : m_in[k];
                v_out[k] = in ? bf16_store<SR>(v[k], SR ? hash32((idx + k) ^ s.seed_v) : 0u) : v_in[k];
            }
            l_out |= ((p_out[k] >> 8) & 0xffu) << (8 * k);
        }
        st(reinterpret_cast<u32x2*>(dst + at_h),
           u32x2{(p_out[0] >> 16) | (p_out[1] & 0xffff0000u), (p_out[2] >> 16) | (p_out[3] & 0xffff0000u)});
        st(reinterpret_cast<uint32_t*>(dst + at_l), l_out);
        if constexpr (kF32) {
            st(reinterpret_cast<u32x4*>(dst + at_m), u32x4{m_out[0], m_out[1], m_out[2], m_out[3]});
            st(reinterpret_cast<u32x4*>(dst + at_v), u32x4{v_out[0], v_out[1], v_out[2], v_out[3]});
        } else {
            st(reinterpret_cast<u32x2*>(dst + at_m), u32x2{m_out[0] | (m_out[1] << 16), m_out[2] | (m_out[3] << 16)});
            st(reinterpret_cast<u32x2*>(dst + at_v), u32x2{v_out[0] | (v_out[1] << 16), v_out[2] | (v_out[3] << 16)});
        }
        if (!prev) store_quad_out<OT>(s.out, i, n, vec && all, p_out);
    }
}

template <int GT, int OT>
__global__ __launch_bounds__(kThreads) void k_update_f24rec(Launch L)
{
    const int64_t tile = block_tile(L);
    if (tile >= L.ntiles) return;
    const DevSeg s = find_segment(L, tile);
    if (s.flags & kSR) update_tile_f24rec<GT, OT, true>(s, tile, L.tile);
    else update_tile_f24rec<GT, OT, false>(s, tile, L.tile);
}

// FP32 moments: only the master rounds (stochastically under kSR).
template <int GT, int OT>
__global__ __launch_bounds__(kThreads) void k_update_f24f32rec(Launch L)
{
    const int64_t tile = block_tile(L);
    if (tile >= L.ntiles) return;
    const DevSeg s = find_segment(L, tile);
    if (s.flags & kSR) update_tile_f24rec<GT, OT, true, DT_F32>(s, tile, L.tile);
    else update_tile_f24rec<GT, OT, false, DT_F32>(s, tile, L.tile);
}

// Lion with an FP24 master and a BF16 moment in one 1280-byte record per 256 elements: the
// record's 256 master high halves, its 256 low bytes and its 256 m values, each in element order.
// The Lion-record kernel's lanes and arithmetic, with the FP24-master records' master access.
// With an FP32 moment (MV = DT_F32, ADAMBRIDGE_DT_PACKED_LION_F24_F32): 1792-byte records, the m
// values FP32 at 768 + 4j (a 16-byte access a lane), stored exactly.
constexpr int64_t kLionF24RecordBytes = 1280;
constexpr int64_t kLionF24F32RecordBytes = 1792;

template <int GT, int OT, bool SR, int MV = DT_BF16>
__device__ __forceinline__ void update_tile_lion_f24rec(const DevSeg& s, int64_t tile, int64_t T)
{
    constexpr bool kF32 = MV == DT_F32;
    constexpr int64_t kRecB = kF32 ? kLionF24F32RecordBytes : kLionF24RecordBytes;
    const int64_t n = s.n;
    const Coef c = s.c;
    const uint8_t* __restrict__ src = static_cast<const uint8_t*>(s.p);
    uint8_t* __restrict__ dst = s.p_lo;
    const bool vec = (s.flags & kVec) != 0;   // g and out allow 2-element access
    const bool prev = (s.flags & kPrev) != 0;  // uniform: out from the master as loaded
    const int64_t lo = (tile - s.tile_begin) * T;
    const int64_t hi = lo + T < n ? lo + T : n;
    for (int64_t i = lo + threadIdx.x * 4; i < hi; i += kThreads * 4) {
        // i % 4 == 0: record i / 256; high halves at 2j, low bytes at 512 + j, m at 768 + 2j (BF16)
        // or 768 + 4j (FP32)
        const int64_t rec = (i / kF24RecordElems) * kRecB;
        const int64_t j = i % kF24RecordElems;
        const int64_t at_h = rec + 2 * j, at_l = rec + 512 + j, at_m = rec + 768 + (kF32 ? 4 : 2) * j;
        const uint32_t idx = s.idx0 + (uint32_t)i;
        const u32x2 hw = ld(reinterpret_cast<const u32x2*>(src + at_h));
        const uint32_t lw = ld(reinterpret_cast<const uint32_t*>(src + at_l));
        uint32_t m_in[4];
        if constexpr (kF32) {
            const u32x4 mw = ld(reinterpret_cast<const u32x4*>(src + at_m));
            m_in[0] = mw.x; m_in[1] = mw.y; m_in[2] = mw.z; m_in[3] = mw.w;
        } else {
            const u32x2 mw = ld(reinterpret_cast<const u32x2*>(src + at_m));
            m_in[0] = mw.x & 0xffffu; m_in[1] = mw.x >> 16; m_in[2] = mw.y & 0xffffu; m_in[3] = mw.y >> 16;
        }
        const bool all = i + 4 <= n;
        float g[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (vec && all) {
            load2<GT>(s.g, i, g[0], g[1]);
            load2<GT>(s.g, i + 2, g[2], g[3]);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (i + k < n) g[k] = load1<GT>(s.g, i + k);
        }
        const uint32_t h_in[4] = {hw.x & 0xffffu, hw.x >> 16, hw.y & 0xffffu, hw.y >> 16};
        uint32_t p_in[4];   // the stored masters as FP32 bits: hi << 16 | lo << 8
#pragma unroll
        for (int k = 0; k < 4; ++k) p_in[k] = (h_in[k] << 16) | (((lw >> (8 * k)) & 0xffu) << 8);
        if (prev) store_quad_out<OT>(s.out, i, n, vec && all, p_in);
        uint32_t p_out[4], m_out[4], l_out = 0u;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float m = bitsf(kF32 ? m_in[k] : m_in[k] << 16);
            const float p = lion(bitsf(p_in[k]), g[k], m, c);
            const bool in = all || i + k < n;   // padding keeps its bits
            p_out[k] = in ? f24_round<SR>(p, SR ? hash32((idx + k) ^ s.seed_p) : 0u) : p_in[k];
            if constexpr (kF32) m_out[k] = in ? fbits(m) : m_in[k];
            else m_out[k] = in ? bf16_store<SR>(m, SR ? hash32((idx + k) ^ s.seed_m) : 0u) : m_in[k];
            l_out |= ((p_out[k] >> 8) & 0xffu) << (8 * k);
        }
        st(reinterpret_cast<u32x2*>(dst + at_h),
           u32x2{(p_out[0] >> 16) | (p_out[1] & 0xffff0000u), (p_out[2] >> 16) | (p_out[3] & 0xffff0000u)});
        st(reinterpret_cast<uint32_t*>(dst + at_l), l_out);
        if constexpr (kF32) st(reinterpret_cast<u32x4*>(dst + at_m), u32x4{m_out[0], m_out[1], m_out[2], m_out[3]});
        else st(reinterpret_cast<u32x2*>(dst + at_m), u32x2{m_out[0] | (m_out[1] << 16), m_out[2] | (m_out[3] << 16)});
        if (!prev) store_quad_out<OT>(s.out, i, n, vec && all, p_out);
    }
}

template <int GT, int OT>
__global__ __launch_bounds__(kThreads) void k_update_lion_f24rec(Launch L)
{
    const int64_t tile = block_tile(L);
    if (tile >= L.ntiles) return;
    const DevSeg s = find_segment(L, tile);
    if (s.flags & kSR) update_tile_lion_f24rec<GT, OT, true>(s, tile, L.tile);
    else update_tile_lion_f24rec<GT, OT, false>(s, tile, L.tile);
}

// FP32 moment: only the master rounds (stochastically under kSR).
template <int GT, int OT>
__global__ __launch_bounds__(kThreads) void k_update_lion_f24f32rec(Launch L)
{
    const int64_t tile = block_tile(L);
    if (tile >= L.ntiles) return;
    const DevSeg s = find_segment(L, tile);
    if (s.flags & kSR) update_tile_lion_f24rec<GT, OT, true, DT_F32>(s, tile, L.tile);
    else update_tile_lion_f24rec<GT, OT, false, DT_F32>(s, tile, L.tile);
}

// ------------------------------------------------------- segment-table writer
//
// The allocation-free entry point keeps its segment tables in a device array
// of the library (no staging buffer, no copy from host memory): each table is
// written by launches of this kernel, the descriptors travelling in its
// kernel arguments, ordered on the stream before the update that reads them.

constexpr int kWriteSegs = 20;   // descriptors per writer launch: 20 x 144 + 24 bytes of arguments

struct TableChunk {
    DevSeg* table;        // destination: table entries [0, count)
    int64_t* starts;      // destination: first tile of each entry
    int32_t count;
    int32_t pad;
    DevSeg segs[kWriteSegs];
};
static_assert(sizeof(TableChunk) <= 4096 - 256, "kernel argument block");

__global__ __launch_bounds__(64) void k_write_table(TableChunk C)
{
    constexpr int kWords = sizeof(DevSeg) / 8;
    const uint64_t* src = reinterpret_cast<const uint64_t*>(&C.segs[0]);
    uint64_t* dst = reinterpret_cast<uint64_t*>(C.table);
    for (int w = threadIdx.x; w < C.count * kWords; w += 64) dst[w] = src[w];
    for (int i = threadIdx.x; i < C.count; i += 64) C.starts[i] = C.segs[i].tile_begin;
}

// ------------------------------------------------------------- calibration copy
//
// A copy of known size with the update kernels' access type (16-byte non-temporal global loads and
// stores) and tile order (kCopyTile bytes per workgroup, XCD-contiguous), for calibrating hardware
// byte counters (FETCH_SIZE, WRITE_SIZE) against the bytes actually moved, and as the rate a plain
// 1:1 read/write stream reaches on the same bytes.

constexpr int64_t kCopyTile = 4 * 1024;   // one 16-byte load per lane: the fastest 1:1 stream measured

__global__ __launch_bounds__(kThreads) void k_stream_copy(const u32x4* src, u32x4* dst, int64_t n16)
{
    const int64_t ntiles = (n16 * 16 + kCopyTile - 1) / kCopyTile;
    const int64_t b = blockIdx.x;
    const int64_t per = (ntiles + kXcds - 1) / kXcds;
    const int64_t tile = (b % kXcds) * per + b / kXcds;
    if (tile >= ntiles) return;
    const int64_t i = tile * (kCopyTile / 16) + threadIdx.x;
    if (i < n16) st(dst + i, ld(src + i));
}

// ------------------------------------------------------------ kernel table

using KernelFn = void (*)(Launch);

// Index: ((((algo * 3 + mv) * 2 + pt) * 2 + gt) * 3 + ot), with
// mv 0/1/2 = F32/BF16/FP8, pt 0/1 = F32/F24, gt 0/1 = F32/BF16, ot 0/1/2 = NONE/F32/BF16.
constexpr int kNumKernels = 2 * 3 * 2 * 2 * 3;

// WIDE: the FP8 kernels' form for tiles of more than one block per 16-lane group (the other
// kernels have one form).
template <int ALGO, int MVI, int PTI, int GTI, int OTI, bool WIDE>
constexpr KernelFn pick()
{
    constexpr int PT = PTI ? DT_F24 : DT_F32;
    constexpr int GT = GTI ? DT_BF16 : DT_F32;
    constexpr int OT = OTI == 0 ? DT_NONE : OTI == 1 ? DT_F32 : DT_BF16;
    if constexpr (MVI == 2) return &k_update_fp8<ALGO, PT, GT, OT, WIDE>;
    else return &k_update<ALGO, MVI ? DT_BF16 : DT_F32, PT, GT, OT>;
}

template <int I, bool WIDE>
constexpr KernelFn entry()
{
    constexpr int ot = I % 3, gt = (I / 3) % 2, pt = (I / 6) % 2, mv = (I / 12) % 3, algo = I / 36;
    return pick<algo, mv, pt, gt, ot, WIDE>();
}

template <bool WIDE, int... I>
constexpr auto make_table(std::integer_sequence<int, I...>)
{
    return std::array<KernelFn, sizeof...(I)>{entry<I, WIDE>()...};
}

// Packed-state kernels follow the table: index kNumKernels + gt * 3 + ot.
constexpr int kNumPacked = 2 * 3;

template <int I>
constexpr KernelFn packed_entry()
{
    constexpr int ot = I % 3, gt = I / 3;
    return &k_update_packed<gt ? DT_BF16 : DT_F32, ot == 0 ? DT_NONE : ot == 1 ? DT_F32 : DT_BF16>;
}

template <int... I>
constexpr auto make_packed_table(std::integer_sequence<int, I...>)
{
    return std::array<KernelFn, sizeof...(I)>{packed_entry<I>()...};
}

// FP8-record kernels (AdamW) follow: index kNumKernels + kNumPacked + gt * 3 + ot.
template <int I, bool WIDE>
constexpr KernelFn packed8_entry()
{
    constexpr int ot = I % 3, gt = I / 3;
    return &k_update_fp8<ALGO_ADAMW, DT_PACKED8, gt ? DT_BF16 : DT_F32, ot == 0 ? DT_NONE : ot == 1 ? DT_F32 : DT_BF16,
                         WIDE>;
}

template <bool WIDE, int... I>
constexpr auto make_packed8_table(std::integer_sequence<int, I...>)
{
    return std::array<KernelFn, sizeof...(I)>{packed8_entry<I, WIDE>()...};
}

// Lion-record kernels follow: index kNumKernels + 2 * kNumPacked + gt * 3 + ot.
template <int I>
constexpr KernelFn lion_rec_entry()
{
    constexpr int ot = I % 3, gt = I / 3;
    return &k_update_lion_rec<gt ? DT_BF16 : DT_F32, ot == 0 ? DT_NONE : ot == 1 ? DT_F32 : DT_BF16>;
}

template <int... I>
constexpr auto make_lion_rec_table(std::integer_sequence<int, I...>)
{
    return std::array<KernelFn, sizeof...(I)>{lion_rec_entry<I>()...};
}

static const auto kKernels = make_table<false>(std::make_integer_sequence<int, kNumKernels>{});
static const auto kKernelsWide = make_table<true>(std::make_integer_sequence<int, kNumKernels>{});
static const auto kPacked = make_packed_table(std::make_integer_sequence<int, kNumPacked>{});
static const auto kPacked8 = make_packed8_table<false>(std::make_integer_sequence<int, kNumPacked>{});
static const auto kPacked8Wide = make_packed8_table<true>(std::make_integer_sequence<int, kNumPacked>{});
static const auto kLionRec = make_lion_rec_table(std::make_integer_sequence<int, kNumPacked>{});

// FP32-moment record kernels (AdamW) follow: index kNumKernels + 3 * kNumPacked + gt * 3 + ot.
template <int I>
constexpr KernelFn f32rec_entry()
{
    constexpr int ot = I % 3, gt = I / 3;
    return &k_update_f32rec<gt ? DT_BF16 : DT_F32, ot == 0 ? DT_NONE : ot == 1 ? DT_F32 : DT_BF16>;
}

template <int... I>
constexpr auto make_f32rec_table(std::integer_sequence<int, I...>)
{
    return std::array<KernelFn, sizeof...(I)>{f32rec_entry<I>()...};
}

static const auto kF32Rec = make_f32rec_table(std::make_integer_sequence<int, kNumPacked>{});

// FP24-master record kernels (AdamW) follow: index kNumKernels + 4 * kNumPacked + gt * 3 + ot.
template <int I>
constexpr KernelFn f24rec_entry()
{
    constexpr int ot = I % 3, gt = I / 3;
    return &k_update_f24rec<gt ? DT_BF16 : DT_F32, ot == 0 ? DT_NONE : ot == 1 ? DT_F32 : DT_BF16>;
}

template <int... I>
constexpr auto make_f24rec_table(std::integer_sequence<int, I...>)
{
    return std::array<KernelFn, sizeof...(I)>{f24rec_entry<I>()...};
}

static const auto kF24Rec = make_f24rec_table(std::make_integer_sequence<int, kNumPacked>{});

// Lion FP24-master record kernels follow: index kNumKernels + 5 * kNumPacked + gt * 3 + ot.
template <int I>
constexpr KernelFn lion_f24rec_entry()
{
    constexpr int ot = I % 3, gt = I / 3;
    return &k_update_lion_f24rec<gt ? DT_BF16 : DT_F32, ot == 0 ? DT_NONE : ot == 1 ? DT_F32 : DT_BF16>;
}

template <int... I>
constexpr auto make_lion_f24rec_table(std::integer_sequence<int, I...>)
{
    return std::array<KernelFn, sizeof...(I)>{lion_f24rec_entry<I>()...};
}

static const auto kLionF24Rec = make_lion_f24rec_table(std::make_integer_sequence<int, kNumPacked>{});

// FP8 records with an FP24 master (AdamW) follow: index kNumKernels + 6 * kNumPacked + gt * 3 + ot.
template <int I, bool WIDE>
constexpr KernelFn packed8_f24_entry()
{
    constexpr int ot = I % 3, gt = I / 3;
    return &k_update_fp8<ALGO_ADAMW, DT_PACKED8_F24, gt ? DT_BF16 : DT_F32, ot == 0 ? DT_NONE : ot == 1 ? DT_F32 : DT_BF16,
                         WIDE>;
}

template <bool WIDE, int... I>
constexpr auto make_packed8_f24_table(std::integer_sequence<int, I...>)
{
    return std::array<KernelFn, sizeof...(I)>{packed8_f24_entry<I, WIDE>()...};
}

static const auto kPacked8F24 = make_packed8_f24_table<false>(std::make_integer_sequence<int, kNumPacked>{});
static const auto kPacked8F24Wide = make_packed8_f24_table<true>(std::make_integer_sequence<int, kNumPacked>{});

// Lion FP32-moment record kernels follow: index kNumKernels + 7 * kNumPacked + gt * 3 + ot.
template <int I>
constexpr KernelFn lion_f32rec_entry()
{
    constexpr int ot = I % 3, gt = I / 3;
    return &k_update_lion_f32rec<gt ? DT_BF16 : DT_F32, ot == 0 ? DT_NONE : ot == 1 ? DT_F32 : DT_BF16>;
}

template <int... I>
constexpr auto make_lion_f32rec_table(std::integer_sequence<int, I...>)
{
    return std::array<KernelFn, sizeof...(I)>{lion_f32rec_entry<I>()...};
}

static const auto kLionF32Rec = make_lion_f32rec_table(std::make_integer_sequence<int, kNumPacked>{});

// Lion FP8 records follow: index kNumKernels + 8 * kNumPacked + gt * 3 + ot.
template <int I, bool WIDE>
constexpr KernelFn packed8_lion_entry()
{
    constexpr int ot = I % 3, gt = I / 3;
    return &k_update_fp8<ALGO_LION, DT_PACKED8_LION, gt ? DT_BF16 : DT_F32, ot == 0 ? DT_NONE : ot == 1 ? DT_F32 : DT_BF16,
                         WIDE>;
}

template <bool WIDE, int... I>
constexpr auto make_packed8_lion_table(std::integer_sequence<int, I...>)
{
    return std::array<KernelFn, sizeof...(I)>{packed8_lion_entry<I, WIDE>()...};
}

static const auto kPacked8Lion = make_packed8_lion_table<false>(std::make_integer_sequence<int, kNumPacked>{});
static const auto kPacked8LionWide = make_packed8_lion_table<true>(std::make_integer_sequence<int, kNumPacked>{});

// FP24-master FP32-moment records (AdamW) follow: index kNumKernels + 9 * kNumPacked + gt * 3 + ot.
template <int I>
constexpr KernelFn f24f32rec_entry()
{
    constexpr int ot = I % 3, gt = I / 3;
    return &k_update_f24f32rec<gt ? DT_BF16 : DT_F32, ot == 0 ? DT_NONE : ot == 1 ? DT_F32 : DT_BF16>;
}

template <int... I>
constexpr auto make_f24f32rec_table(std::integer_sequence<int, I...>)
{
    return std::array<KernelFn, sizeof...(I)>{f24f32rec_entry<I>()...};
}

static const auto kF24F32Rec = make_f24f32rec_table(std::make_integer_sequence<int, kNumPacked>{});

// Lion FP24-master FP32-moment records follow: index kNumKernels + 10 * kNumPacked + gt * 3 + ot.
template <int I>
constexpr KernelFn lion_f24f32rec_entry()
{
    constexpr int ot = I % 3, gt = I / 3;
    return &k_update_lion_f24f32rec<gt ? DT_BF16 : DT_F32, ot == 0 ? DT_NONE : ot == 1 ? DT_F32 : DT_BF16>;
}

template <int... I>
constexpr auto make_lion_f24f32rec_table(std::integer_sequence<int, I...>)
{
    return std::array<KernelFn, sizeof...(I)>{lion_f24f32rec_entry<I>()...};
}

static const auto kLionF24F32Rec = make_lion_f24f32rec_table(std::make_integer_sequence<int, kNumPacked>{});

// Lion FP8 records with an FP24 master follow: index kNumKernels + 11 * kNumPacked + gt * 3 + ot.
template <int I, bool WIDE>
constexpr KernelFn packed8_lion_f24_entry()
{
    constexpr int ot = I % 3, gt = I / 3;
    return &k_update_fp8<ALGO_LION, DT_PACKED8_LION_F24, gt ? DT_BF16 : DT_F32,
                         ot == 0 ? DT_NONE : ot == 1 ? DT_F32 : DT_BF16, WIDE>;
}

template <bool WIDE, int... I>
constexpr auto make_packed8_lion_f24_table(std::integer_sequence<int, I...>)
{
    return std::array<KernelFn, sizeof...(I)>{packed8_lion_f24_entry<I, WIDE>()...};
}

static const auto kPacked8LionF24 = make_packed8_lion_f24_table<false>(std::make_integer_sequence<int, kNumPacked>{});
static const auto kPacked8LionF24Wide = make_packed8_lion_f24_table<true>(std::make_integer_sequence<int, kNumPacked>{});

// Kernel family of a table index: the FP8 block kernel, or a two-element-per-lane kernel.
inline bool kernel_is_fp8(int index)
{
    if (index < kNumKernels) return (index / 12) % 3 == 2;
    return (index >= kNumKernels + kNumPacked && index < kNumKernels + 2 * kNumPacked) ||
           (index >= kNumKernels + 6 * kNumPacked && index < kNumKernels + 7 * kNumPacked) ||
           (index >= kNumKernels + 8 * kNumPacked && index < kNumKernels + 9 * kNumPacked) ||
           (index >= kNumKernels + 11 * kNumPacked && index < kNumKernels + 12 * kNumPacked);
}

// Dynamic LDS (unused) per workgroup of a launch of kernel `index`: it caps the workgroups a CU holds
// (160 KiB of LDS per CU).  These kernels need 45-58 VGPRs, which would allow 8 workgroups (32
// wavefronts) per CU; with 6 the AdamW FP8 kernels with an FP32 master and the FP32-record kernel
// move their bytes faster.  Measured on MI355X through bench.py's path (arena-placed state, one
// launch per step; ms per launch, two passes each, interleaved in one process):
//   - FP8 records, the 7B list (291 tensors): 6 workgroups per CU 17.62-17.70, 8: 17.82-17.97,
//     5: 18.01-18.04;
//   - FP32 records, the 7B list: 6: 29.35, 8: 29.46-29.50, 5: 29.44-29.50;
//   - FP32 records, one 16.8M-element tensor (512-element tiles, two active wavefronts per
//     workgroup; a lone launch, interleaved): 6: 0.078, 8: 0.085, 5: 0.087.
// Lion records at the 1.5B list (338 tensors) run alike with 6 or 8 (4.00-4.03) and lose 13% with 5
// (4.58-4.61): the segment search each workgroup makes first is hidden by fewer others there.  Lion
// records with an FP32 moment (family 7) gain from 6: 1.54G elements in 8 tensors 4.98 ms against
// 5.09 at 7 and 5.15 at 8; 6.74G elements 21.02 against 21.17 and 21.38.  Lion with an FP8 moment
// in separate arrays (1.54G elements in 8 tensors) is fastest at 5 with an FP32 master (3.68-3.71 ms;
// 4: 3.70, 3: 3.74, 6: 3.89, 8: 3.97, 2: 4.58) and at 6 with an FP24 master (3.15 ms; 5 and 4:
// 3.18, 8: 3.21).  Lion FP8 records: 5 per CU 3.51 ms, 4: 3.50, 6: 3.69, 8: 3.75.  FP24-master
// FP32-moment records (6.74G elements in 8 tensors): 5 per CU 27.12 ms (the copy of their bytes:
// 27.14), 6: 27.73, 8: 27.93.  Lion FP8 records with an FP24 master: 6 per CU 3.04 ms, 4: 3.10,
// 5: 3.11, 8: 3.12.  The
// BF16 pairs lose with fewer workgroups (the 0.5B list: 1.76 against 1.67 ms with 6), and the
// FP24-master FP8 kernels keep 8 (records, the 7B list: 8 per CU 16.28-16.66, 7: 16.18-16.55, 6:
// 16.44-16.65, 5: 17.56-17.91).  Those run at the speed of their accesses alone: a form that makes
// the same loads and stores and no arithmetic took 16.45 ms at 8 per CU, and its time falls as the
// CU holds fewer workgroups (15.46 at 5, 15.15 at 3) while the arithmetic needs the wavefronts.
inline size_t launch_lds(int index)
{
    constexpr size_t kCap6 = 24 * 1024;   // 6 workgroups of 24 KiB in 160 KiB; 7 would need 168
    constexpr size_t kCap5 = 32 * 1024;   // 5 of 32 KiB; 6 would need 192
    if (index < kNumKernels) {
        const int pt = (index / 6) % 2, mv = (index / 12) % 3, algo = index / 36;
        if (mv != 2) return 0;   // FP8 moments only
        if (algo == ALGO_ADAMW) return pt == 0 ? kCap6 : 0;
        return pt == 0 ? kCap5 : kCap6;   // Lion: FP32 / FP24 master
    }
    // 1: FP8 records, 3: FP32 records, 7: Lion records with an FP32 moment, 8: Lion FP8 records,
    // 9: FP24-master FP32-moment records, 10: their Lion form, 11: Lion FP8 records with an FP24 master
    const int family = (index - kNumKernels) / kNumPacked;
    if (family == 8 || family == 9) return kCap5;
    if (family == 10 || family == 11) return kCap6;
    return family == 1 || family == 3 || family == 7 ? kCap6 : 0;
}

// The FP8 kernels' form for tiles of more than one block per 16-lane group (kernel_is_fp8(index)).
inline KernelFn wide_kernel_at(int index)
{
    if (index < kNumKernels) return kKernelsWide[index];
    if (index < kNumKernels + 2 * kNumPacked) return kPacked8Wide[index - kNumKernels - kNumPacked];
    if (index < kNumKernels + 7 * kNumPacked) return kPacked8F24Wide[index - kNumKernels - 6 * kNumPacked];
    if (index < kNumKernels + 9 * kNumPacked) return kPacked8LionWide[index - kNumKernels - 8 * kNumPacked];
    return kPacked8LionF24Wide[index - kNumKernels - 11 * kNumPacked];
}

inline KernelFn kernel_at(int index)
{
    if (index < kNumKernels) return kKernels[index];
    if (index < kNumKernels + kNumPacked) return kPacked[index - kNumKernels];
    if (index < kNumKernels + 2 * kNumPacked) return kPacked8[index - kNumKernels - kNumPacked];
    if (index < kNumKernels + 3 * kNumPacked) return kLionRec[index - kNumKernels - 2 * kNumPacked];
    if (index < kNumKernels + 4 * kNumPacked) return kF32Rec[index - kNumKernels - 3 * kNumPacked];
    if (index < kNumKernels + 5 * kNumPacked) return kF24Rec[index - kNumKernels - 4 * kNumPacked];
    if (index < kNumKernels + 6 * kNumPacked) return kLionF24Rec[index - kNumKernels - 5 * kNumPacked];
    if (index < kNumKernels + 7 * kNumPacked) return kPacked8F24[index - kNumKernels - 6 * kNumPacked];
    if (index < kNumKernels + 8 * kNumPacked) return kLionF32Rec[index - kNumKernels - 7 * kNumPacked];
    if (index < kNumKernels + 9 * kNumPacked) return kPacked8Lion[index - kNumKernels - 8 * kNumPacked];
    if (index < kNumKernels + 10 * kNumPacked) return kF24F32Rec[index - kNumKernels - 9 * kNumPacked];
    if (index < kNumKernels + 11 * kNumPacked) return kLionF24F32Rec[index - kNumKernels - 10 * kNumPacked];
    return kPacked8LionF24[index - kNumKernels - 11 * kNumPacked];
}

inline int kernel_index(int algo, int mv, int pt, int gt, int ot)
{
    if (pt == DT_PACKED)
        return kNumKernels + (gt == DT_BF16 ? 1 : 0) * 3 + (ot == DT_NONE ? 0 : ot == DT_F32 ? 1 : 2);
    if (pt == DT_PACKED8)
        return kNumKernels + kNumPacked + (gt == DT_BF16 ? 1 : 0) * 3 + (ot == DT_NONE ? 0 : ot == DT_F32 ? 1 : 2);
    if (pt == DT_PACKED_LION)
        return kNumKernels + 2 * kNumPacked + (gt == DT_BF16 ? 1 : 0) * 3 + (ot == DT_NONE ? 0 : ot == DT_F32 ? 1 : 2);
    if (pt == DT_PACKED_F32)
        return kNumKernels + 3 * kNumPacked + (gt == DT_BF16 ? 1 : 0) * 3 + (ot == DT_NONE ? 0 : ot == DT_F32 ? 1 : 2);
    if (pt == DT_PACKED_F24)
        return kNumKernels + 4 * kNumPacked + (gt == DT_BF16 ? 1 : 0) * 3 + (ot == DT_NONE ? 0 : ot == DT_F32 ? 1 : 2);
    if (pt == DT_PACKED_LION_F24)
        return kNumKernels + 5 * kNumPacked + (gt == DT_BF16 ? 1 : 0) * 3 + (ot == DT_NONE ? 0 : ot == DT_F32 ? 1 : 2);
    if (pt == DT_PACKED8_F24)
        return kNumKernels + 6 * kNumPacked + (gt == DT_BF16 ? 1 : 0) * 3 + (ot == DT_NONE ? 0 : ot == DT_F32 ? 1 : 2);
    if (pt == DT_PACKED_LION_F32)
        return kNumKernels + 7 * kNumPacked + (gt == DT_BF16 ? 1 : 0) * 3 + (ot == DT_NONE ? 0 : ot == DT_F32 ? 1 : 2);
    if (pt == DT_PACKED8_LION)
        return kNumKernels + 8 * kNumPacked + (gt == DT_BF16 ? 1 : 0) * 3 + (ot == DT_NONE ? 0 : ot == DT_F32 ? 1 : 2);
    if (pt == DT_PACKED_F24_F32)
        return kNumKernels + 9 * kNumPacked + (gt == DT_BF16 ? 1 : 0) * 3 + (ot == DT_NONE ? 0 : ot == DT_F32 ? 1 : 2);
    if (pt == DT_PACKED_LION_F24_F32)
        return kNumKernels + 10 * kNumPacked + (gt == DT_BF16 ? 1 : 0) * 3 + (ot == DT_NONE ? 0 : ot == DT_F32 ? 1 : 2);
    if (pt == DT_PACKED8_LION_F24)
        return kNumKernels + 11 * kNumPacked + (gt == DT_BF16 ? 1 : 0) * 3 + (ot == DT_NONE ? 0 : ot == DT_F32 ? 1 : 2);
    const int mvi = mv == DT_F32 ? 0 : mv == DT_BF16 ? 1 : 2;
    const int pti = pt == DT_F24 ? 1 : 0;
    const int gti = gt == DT_BF16 ? 1 : 0;
    const int oti = ot == DT_NONE ? 0 : ot == DT_F32 ? 1 : 2;
    return (((algo * 3 + mvi) * 2 + pti) * 2 + gti) * 3 + oti;
}

// ----------------------------------------------------- storage conversion kernel

// Re-encoding of one moment (or an FP32 master) between storage formats, the device form of the
// reference's torch-side stores (precision.py:341-418): values decoded exactly (FP8: code x
// scale, squared for the sqrt-domain v), then encoded to nearest: BF16, or FP8 per 128-element
// block with v = sqrt(clamp(v, min=0)), scale = absmax / format max (1 for an all-zero block, and,
// as torch's amax propagates NaN, for a block holding a NaN), codes of clamp(x / scale, +-max).
// NaN encodes as torch's casts encode it: BF16 0x7fc0, FP8 0x7f with the value's sign (E5M2
// included, where the update kernel's code is 0x7e).  Positions past n encode as zero (padding).
// 16 lanes per block, element b0 + 16k + lane for k < 8: every access of the 16 lanes is
// contiguous.
template <int SRC, int DST, bool V>
__global__ __launch_bounds__(kThreads) void k_convert(const void* src, const float* src_scale, void* dst,
                                                      float* dst_scale, int64_t n)
{
    const int64_t nb = (n + kFp8Block - 1) / kFp8Block;
    const int64_t blk = (int64_t)blockIdx.x * (kThreads / 16) + (threadIdx.x >> 4);
    if (blk >= nb) return;   // a 16-lane group leaves whole: the shuffles below stay within live groups
    const int lane = threadIdx.x & 15;
    const int64_t b0 = blk * kFp8Block;
    float x[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int64_t e = b0 + 16 * k + lane;
        float val = 0.0f;
        if constexpr (SRC == DT_FP8) {   // codes exist for the whole padded block
            const uint32_t code = ld(static_cast<const uint8_t*>(src) + e);
            const float u = (V ? e5m2_decode<0>(code) : e4m3_decode<0>(code)) * ld(src_scale + blk);
            val = V ? u * u : u;
            if (e >= n) val = 0.0f;
        } else if (e < n) {
            if constexpr (SRC == DT_BF16) val = bitsf((uint32_t)ld(static_cast<const uint16_t*>(src) + e) << 16);
            else val = ld(static_cast<const float*>(src) + e);
        }
        x[k] = val;
    }
    if constexpr (DST == DT_F32 || DST == DT_BF16) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int64_t e = b0 + 16 * k + lane;
            if (e >= n) continue;
            if constexpr (DST == DT_F32) st(static_cast<float*>(dst) + e, x[k]);
            else st(static_cast<uint16_t*>(dst) + e, (uint16_t)(x[k] != x[k] ? 0x7fc0u : bf16_rne(x[k])));
        }
    } else {
        constexpr float kMax = V ? 57344.0f : 448.0f;
        float amax = 0.0f;
        int nan = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if constexpr (V) x[k] = __builtin_sqrtf(x[k] < 0.0f ? 0.0f : x[k]);   // NaN and -0 pass through
            const float a = fabsf(x[k]);
            nan |= a != a;
            amax = a > amax ? a : amax;
        }
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) {
            amax = fmaxf(amax, __shfl_xor(amax, d, 16));
            nan |= __shfl_xor(nan, d, 16);
        }
        const float scale = (!nan && amax > 0.0f) ? amax / kMax : 1.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            float y = x[k] / scale;
            y = y > kMax ? kMax : (y < -kMax ? -kMax : y);   // NaN passes
            const uint32_t code = y != y ? ((fbits(y) >> 24) & 0x80u) | 0x7fu
                                         : V ? e5m2_encode<false>(y, 0u) : e4m3_encode<false>(y, 0u);
            st(static_cast<uint8_t*>(dst) + b0 + 16 * k + lane, (uint8_t)code);
        }
        if (lane == 0) st(dst_scale + blk, scale);
    }
}

using ConvertFn = void (*)(const void*, const float*, void*, float*, int64_t);

template <int SRC, int DST>
constexpr ConvertFn convert_for(bool v)
{
    return v ? &k_convert<SRC, DST, true> : &k_convert<SRC, DST, false>;
}

inline ConvertFn convert_kernel(int src, int dst, bool v)
{
    const int si = src == DT_F32 ? 0 : src == DT_BF16 ? 1 : 2, di = dst == DT_F32 ? 0 : dst == DT_BF16 ? 1 : 2;
    switch (si * 3 + di) {
    case 0: return convert_for<DT_F32, DT_F32>(v);
    case 1: return convert_for<DT_F32, DT_BF16>(v);
    case 2: return convert_for<DT_F32, DT_FP8>(v);
    case 3: return convert_for<DT_BF16, DT_F32>(v);
    case 4: return convert_for<DT_BF16, DT_BF16>(v);
    case 5: return convert_for<DT_BF16, DT_FP8>(v);
    case 6: return convert_for<DT_FP8, DT_F32>(v);
    case 7: return convert_for<DT_FP8, DT_BF16>(v);
    default: return convert_for<DT_FP8, DT_FP8>(v);
    }
}

// --------------------------------------------------------- plane conversion kernel
//
// Master weights (or any FP32 / BF16 / FP24 values) from one plane to another: the FP24 master's
// rounding on load (kernels.c:145-160; precision.py:421-480), its expansion to FP32, and the bf16
// working weight of a master (kernels.c:108-112), each in one pass with no temporaries.  A plane
// is a base address and a group structure: element i lives at data + (i >> shift) * stride +
// (i & (2^shift - 1)) * size (stride 0: contiguous), which describes the separate arrays and the
// master columns of the interleaved layouts alike; DT_PACKED8 names the masters of FP8 block
// records (record_master_offset), the stride then the record size.  One element per lane, grid-stride.

struct DevPlane {
    uint8_t* data;
    uint8_t* lo;
    int64_t stride;
    int32_t dtype;
    int32_t shift;
};

// Byte offset of element i in plane q for values of `size` bytes.
__device__ __forceinline__ int64_t plane_at(const DevPlane& q, int64_t i, int64_t size)
{
    if (q.stride == 0) return i * size;
    return (i >> q.shift) * q.stride + (i & (((int64_t)1 << q.shift) - 1)) * size;
}

// The FP32 bits of element i of a plane of type DT.
template <int DT>
__device__ __forceinline__ uint32_t plane_load(const DevPlane& q, int64_t i)
{
    if constexpr (DT == DT_F32) return ld(reinterpret_cast<const uint32_t*>(q.data + plane_at(q, i, 4)));
    else if constexpr (DT == DT_PACKED8) return ld(reinterpret_cast<const uint32_t*>(q.data + record_master_offset(i, q.stride)));
    else if constexpr (DT == DT_BF16) return (uint32_t)ld(reinterpret_cast<const uint16_t*>(q.data + plane_at(q, i, 2))) << 16;
    else
        return ((uint32_t)ld(reinterpret_cast<const uint16_t*>(q.data + plane_at(q, i, 2))) << 16) |
               ((uint32_t)ld(q.lo + plane_at(q, i, 1)) << 8);
}

// FP32 bits b stored as element i of a plane of type DT; `exact`: b is representable in DT
// (copied bit for bit), else rounded -- stochastically with r when SR, to nearest otherwise.
template <int DT, bool SR>
__device__ __forceinline__ void plane_store(const DevPlane& q, int64_t i, uint32_t b, bool exact, uint32_t r)
{
    if constexpr (DT == DT_F32) st(reinterpret_cast<uint32_t*>(q.data + plane_at(q, i, 4)), b);
    else if constexpr (DT == DT_PACKED8) st(reinterpret_cast<uint32_t*>(q.data + record_master_offset(i, q.stride)), b);
    else if constexpr (DT == DT_BF16) {
        const uint32_t h = exact ? b >> 16 : bf16_store<SR>(bitsf(b), r);   // nearest: the working weight's rule
        st(reinterpret_cast<uint16_t*>(q.data + plane_at(q, i, 2)), (uint16_t)h);
    } else {
        const uint32_t t = exact ? b : f24_round<SR>(bitsf(b), r);
        st(reinterpret_cast<uint16_t*>(q.data + plane_at(q, i, 2)), (uint16_t)(t >> 16));
        st(q.lo + plane_at(q, i, 1), (uint8_t)(t >> 8));
    }
}

// Whether every value of type SRC is representable in type DST.
constexpr bool plane_exact(int src, int dst)
{
    const int w = [](int d) { return d == DT_BF16 ? 16 : d == DT_F24 ? 24 : 32; }(src);
    const int v = [](int d) { return d == DT_BF16 ? 16 : d == DT_F24 ? 24 : 32; }(dst);
    return w <= v;
}

template <int SRC, int DST, bool SR>
__global__ __launch_bounds__(kThreads) void k_convert_plane(DevPlane src, DevPlane dst, int64_t n, uint32_t idx0,
                                                            uint32_t seed)
{
    constexpr bool kExact = plane_exact(SRC, DST);
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        const uint32_t b = plane_load<SRC>(src, i);
        const uint32_t r = (SR && !kExact) ? hash32((idx0 + (uint32_t)i) ^ seed) : 0u;
        plane_store<DST, SR>(dst, i, b, kExact, r);
    }
}

using PlaneFn = void (*)(DevPlane, DevPlane, int64_t, uint32_t, uint32_t);

// Plane types by index: 0 F32, 1 BF16, 2 F24, 3 FP8-record masters.
constexpr int kPlaneTypes[4] = {DT_F32, DT_BF16, DT_F24, DT_PACKED8};

template <int I>
constexpr PlaneFn plane_entry()
{
    constexpr int s = (I / 2) / 4, d = (I / 2) % 4;
    return &k_convert_plane<kPlaneTypes[s], kPlaneTypes[d], (I % 2) == 1>;
}

template <int... I>
constexpr auto make_plane_table(std::integer_sequence<int, I...>)
{
    return std::array<PlaneFn, sizeof...(I)>{plane_entry<I>()...};
}

static const auto kPlaneKernels = make_plane_table(std::make_integer_sequence<int, 32>{});

inline int plane_type_index(int dtype)
{
    return dtype == DT_F32 ? 0 : dtype == DT_BF16 ? 1 : dtype == DT_F24 ? 2 : dtype == DT_PACKED8 ? 3 : -1;
}

// ------------------------------------------------------ conversion self-check

// Every FP32 bit pattern through the conversion instructions the kernels use, compared with the
// integer forms of the reference's rules (fp8_encode, bf16_rne_soft) in the ranges where the
// kernels use the instructions.  counts[c] accumulates the differing results of check c:
// 0 stochastic E4M3, 1 stochastic E5M2, 2 nearest-even E4M3, 3 nearest-even E5M2, 4 BF16,
// 5 square roots (sqrtf on every finite x >= 0, sqrt_mid on its range) against the exact nearest
// root, 6 FP8 decoding (every code of both formats at every byte position:
// packed conversion, NaN detection, per-code conversion) against the formats' definitions,
// 7 divisions (one sampled pair per input: divisions_match) against the exact nearest quotient,
// 8 reciprocals (recip_nearest on every s of its range) against the exact nearest quotient 1 / s.
// The random bits of input x are hash32(x ^ seed); every byte / half-word position is exercised.
constexpr int kConvChecks = 9;

template <bool E5M2>
__device__ __forceinline__ uint32_t sr_code_at(float x, uint32_t r, uint32_t pos)
{
    switch (pos) {
    case 0: return fp8_hw_sr<E5M2, 0>(x, r, 0u) & 0xffu;
    case 1: return (fp8_hw_sr<E5M2, 1>(x, r, 0u) >> 8) & 0xffu;
    case 2: return (fp8_hw_sr<E5M2, 2>(x, r, 0u) >> 16) & 0xffu;
    default: return fp8_hw_sr<E5M2, 3>(x, r, 0u) >> 24;
    }
}

// Whether s is the float nearest to sqrt(x), for finite x >= 0, in exact integer arithmetic
// (no floating-point operation involved): with x = X 2^ex and s = S 2^es (S, X the significands),
// s is nearest iff 16 X 2^(ex - 2 es) lies strictly between (4S - 2)^2 and (4S + 2)^2 -- (4S - 1)^2
// below a power of two, where the float beneath is only half an ulp away.  Ties cannot occur.
__device__ __forceinline__ void float_parts(uint32_t b, uint64_t& m, int& e)
{
    const uint32_t be = (b >> 23) & 0xffu, bm = b & 0x7fffffu;
    m = be ? (bm | 0x800000u) : bm;
    e = be ? (int)be - 150 : -149;
}

__device__ bool is_nearest_root(uint32_t xb, uint32_t sb)
{
    if (xb == 0u) return sb == 0u;
    uint64_t X, S;
    int ex, es;
    float_parts(xb, X, ex);
    float_parts(sb, S, es);
    if (S == 0u || (sb >> 31)) return false;
    typedef unsigned __int128 u128;
    const uint64_t l4 = (S == 0x800000u && es > -149) ? 4 * S - 1 : 4 * S - 2;
    u128 L = (u128)(16 * X), lo = (u128)l4 * l4, hi = (u128)(4 * S + 2) * (4 * S + 2);
    const int k = ex - 2 * es;
    if (k >= 0) {
        if (k > 70) return false;
        L <<= k;
    } else {
        if (-k > 70) return false;
        lo <<= -k;
        hi <<= -k;
    }
    return lo < L && L < hi;
}

// Whether q is the float nearest to a / b, for finite nonzero a, b and a normal q, in exact integer
// arithmetic: 2|a - q b| < ulp(q) |b|, with the bound halved below a power of two (where the float
// beneath q is half an ulp away).
__device__ bool is_nearest_quotient(uint32_t ab, uint32_t bb, uint32_t qb)
{
    if ((qb >> 31) != ((ab ^ bb) >> 31)) return false;
    uint64_t A, B, Q;
    int ea, eb, eq;
    float_parts(ab & 0x7fffffffu, A, ea);
    float_parts(bb & 0x7fffffffu, B, eb);
    float_parts(qb & 0x7fffffffu, Q, eq);
    if (Q < 0x800000u) return false;   // callers keep quotients normal
    typedef unsigned __int128 u128;
    const int ep = eq + eb, e0 = ea < ep ? ea : ep;
    if (ea - e0 > 60 || ep - e0 > 60) return false;
    const u128 x1 = (u128)(4 * A) << (ea - e0), x2 = (u128)(4 * Q * B) << (ep - e0);
    const bool below = x1 < x2;   // a / b below q
    const u128 dist = below ? x2 - x1 : x1 - x2;
    const u128 bound = (u128)((Q == 0x800000u && below) ? B : 2 * B) << (ep - e0);
    return dist < bound;
}

// A float of random significand and sign with exponent in [emin, emax], from two hash draws.
__device__ __forceinline__ float random_float(uint32_t h1, uint32_t h2, int emin, int emax, bool positive)
{
    const uint32_t e = (uint32_t)(emin + (int)(h2 % (uint32_t)(emax - emin + 1)) + 127);
    return bitsf((positive ? 0u : (h2 & 0x80000000u)) | (e << 23) | (h1 & 0x7fffffu));
}

// The divisions the kernels rely on, one sampled pair each per call: the correctly rounded '/'
// of the AdamW step (m / den), and the FP8 block quotients x / scale (block_scale, block_div,
// block_quot_fast, both sign variants).
__device__ bool divisions_match(uint32_t u, uint32_t seed)
{
    const uint32_t h1 = hash32(u ^ seed ^ 0x3c6ef372u), h2 = hash32(h1 ^ 0xa54ff53au);
    const uint32_t h3 = hash32(h2 ^ 0x510e527fu), h4 = hash32(h3 ^ 0x9b05688cu);
    // m / den: |m| in [2^-60, 2^61), den in [2^-50, 2^61) -- '/' everywhere, quot_fast where the
    // AdamW kernels take it (|m| <= 2^60, den below 2^61)
    const float m = random_float(h1, h2, -60, 60, false), den = random_float(h3, h4, -50, 60, true);
    if (!is_nearest_quotient(fbits(m), fbits(den), fbits(m / den))) return false;
    if (quot_m_offset(m) <= kQuotMSpan && !is_nearest_quotient(fbits(m), fbits(den), fbits(quot_fast(m, den))))
        return false;
    // block quotient: absmax in [2^-110, 2^60] (all three paths of block_div), |x| <= absmax
    const float amax = random_float(h2, h3, -110, 60, true);
    const bool e5m2 = h4 & 1u;
    const float s = e5m2 ? block_scale<true>(amax) : block_scale<false>(amax);
    const BlockDiv d = block_div(s, amax);
    const float r = bitsf((h1 & 0x807fffffu) | (126u << 23));   // (-1, -0.5] or [0.5, 1)
    const float x = amax * r;
    if (!(x != 0.0f)) return true;
    const bool plain = (h4 & 2u) != 0u;   // x is nonzero and not NaN here: either variant applies
    float q;
    if (!d.fast) q = x / d.s;
    else if (d.pre == 1.0f) q = plain ? block_quot_fast<false, true>(x, d) : block_quot_fast<false, false>(x, d);
    else q = plain ? block_quot_fast<true, true>(x, d) : block_quot_fast<true, false>(x, d);
    const float aq = fabsf(q);
    if (!(aq >= 0x1p-126f)) return true;   // quotients below the normal range are not asserted here
    return is_nearest_quotient(fbits(x), fbits(s), fbits(q));
}

// Code `code` of format E5M2 (else E4M3FN) placed in byte `pos` of a word with other bytes
// zero: packed and per-code decoders against fp8_value_soft (NaN: a NaN of the code's sign from
// the per-code decoder, which decode_codes takes where the packed conversion gives NaN).
template <bool E5M2>
__device__ __forceinline__ bool decode_matches_fmt(uint32_t code, uint32_t pos)
{
    const uint32_t word = code << (8 * pos);
    float x[8];
    decode_codes<E5M2>(u32x2{word, 0u}, x);
    float y[8];
    decode_codes<E5M2>(u32x2{0u, word}, y);
    const float want = fp8_value_soft<E5M2>(code);
    const float got = x[pos], got_hi = y[4 + pos];
    const bool nan = want != want;
    if (nan) return got != got && got_hi != got_hi && (fbits(got) >> 31) == (code >> 7) && (fbits(got_hi) >> 31) == (code >> 7);
    return fbits(got) == fbits(want) && fbits(got_hi) == fbits(want);
}

__device__ __forceinline__ bool decode_matches(uint32_t code, uint32_t e5m2, uint32_t pos)
{
    return e5m2 ? decode_matches_fmt<true>(code, pos) : decode_matches_fmt<false>(code, pos);
}

__global__ __launch_bounds__(kThreads) void k_check_conversions(unsigned long long* counts, uint32_t seed)
{
    unsigned long long c[kConvChecks] = {0ull, 0ull, 0ull, 0ull, 0ull, 0ull, 0ull, 0ull, 0ull};
    const uint64_t stride = (uint64_t)gridDim.x * kThreads;
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < (1ull << 32); i += stride) {
        const uint32_t u = (uint32_t)i;
        const float x = bitsf(u);
        const uint32_t r = hash32(u ^ seed);
        const uint32_t pos = (u >> 7) & 3u;
        if (fp8_hw_range<false, true>(x) && sr_code_at<false>(x, r, pos) != fp8_encode<3, 7, true>(x, r)) ++c[0];
        if (fp8_hw_range<true, true>(x) && sr_code_at<true>(x, r, pos) != fp8_encode<2, 15, true>(x, r)) ++c[1];
        if (fp8_hw_range<false, false>(x)) {
            const uint32_t w = fp8_hw_rne2<false, true>(x, -x, fp8_hw_rne2<false, false>(-x, x, 0u));
            const uint32_t a = fp8_encode<3, 7, false>(x, 0u), b = fp8_encode<3, 7, false>(-x, 0u);
            if (w != (b | (a << 8) | (a << 16) | (b << 24))) ++c[2];
        }
        if (fp8_hw_range<true, false>(x)) {
            const uint32_t w = fp8_hw_rne2<true, true>(x, -x, fp8_hw_rne2<true, false>(-x, x, 0u));
            const uint32_t a = fp8_encode<2, 15, false>(x, 0u), b = fp8_encode<2, 15, false>(-x, 0u);
            if (w != (b | (a << 8) | (a << 16) | (b << 24))) ++c[3];
        }
        const uint32_t h = bf16x2_rne(x, bitsf(u ^ 0x80000000u));
        if (h != (bf16_rne_soft(x) | (bf16_rne_soft(bitsf(u ^ 0x80000000u)) << 16)) || bf16_rne(x) != bf16_rne_soft(x))
            ++c[4];
        if (u < 0x7f800000u &&   // x >= 0, finite: sqrtf, and the short form on its range, are the nearest root
            (!is_nearest_root(u, fbits(__builtin_sqrtf(x))) || (sqrt_mid_range(x) && !is_nearest_root(u, fbits(sqrt_mid(x))))))
            ++c[5];
        if (i < 2048u && !decode_matches(u & 0xffu, (u >> 8) & 1u, u >> 9)) ++c[6];
        if (!divisions_match(u, seed)) ++c[7];
        if (recip_range(x) && !is_nearest_quotient(0x3f800000u, u, fbits(recip_nearest(x)))) ++c[8];
    }
#pragma unroll
    for (int k = 0; k < kConvChecks; ++k)
        if (c[k]) atomicAdd(&counts[k], c[k]);
}

}  // namespace abh

#include "abh_host.inc"
