// gllm_common.h -- shared device helpers and host plumbing of libgllm_hip.
//
// All HIP sources are compiled with -ffp-contract=off: a fused multiply-add
// appears only where written as fmaf(), matching the VFMADD* sites of the
// reference's amd64 kernels; every other float operation rounds on its own.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <string>

#include "../../include/gllm_hip.h"

namespace gllm {

// ---------------------------------------------------------------------------
// host side: error reporting and per-thread resources
// ---------------------------------------------------------------------------

void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
// Returns GLLM_OK or GLLM_EDEVICE (after recording the message).
int check(hipError_t e, const char* what);

#define GLLM_TRY(expr)                         \
    do {                                       \
        int _rc = (expr);                      \
        if (_rc != GLLM_OK) return _rc;        \
    } while (0)
#define GLLM_HIP(expr) GLLM_TRY(::gllm::check((expr), #expr))

// Per-thread stream used by the blocking host entry points.
hipStream_t thread_stream();
// Per-thread growable device scratch (slot 0..7).
void* thread_scratch(int slot, size_t bytes);
// Per-thread pinned host staging buffer.
void* thread_pinned(int slot, size_t bytes);

// Activation buffers produced by the Q8K quantiser for p rows of cols floats.
struct ActQ8 {
    int8_t* q8perm;  // [p][cols] lane-permuted int8 (see q8perm_offset)
    float* xscale;   // [p][cols/256]
    float* xs32;     // [p][cols/32]   per-32 sums (amd64 order)
    float* xs16;     // [p][cols/16]   per-16 sums x 32 (amd64 order)
    int cols, p;
};
size_t act_bytes(int cols, int p);
void act_carve(void* base, int cols, int p, ActQ8* a);
int launch_q8k_prep(const float* d_x, int cols, int p, const ActQ8& a, hipStream_t s);

struct WeightDesc;  // defined in gemv.hip

}  // namespace gllm

struct gllm_hip_weight {
    int type;
    int rows, cols;
    int blocks;          // cols / 256
    size_t row_bytes;    // reference bytes per row
    uint8_t* d_data;     // device bytes, repacked for Q6_K / Q8_0
    int device;
};

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

namespace gllm {

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    // v_cvt_f32_f16: exact widening (subnormals, Inf, NaN preserved) == the
    // reference's f16LUT (simd.go:73-113).
    _Float16 v;
    uint16_t hb = (uint16_t)h;
    __builtin_memcpy(&v, &hb, 2);
    return (float)v;
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    // v_cvt_f16_f32 under the default round-to-nearest-even mode ==
    // F32ToF16 (kv_f16.go:17-49) for every non-NaN input.
    _Float16 v = (_Float16)f;
    uint16_t hb;
    __builtin_memcpy(&hb, &v, 2);
    return hb;
}

// Byte offset, inside one 256-element block of the lane-permuted Q8K
// activation layout, of element e = 32*m + 4*k + j: lane k of every row
// kernel reads its eight dwords (m = 0..7) as two contiguous 16-byte loads.
__host__ __device__ __forceinline__ int q8perm_offset(int e) {
    int m = e >> 5, k = (e >> 2) & 7, j = e & 3;
    return k * 32 + m * 4 + j;
}

__device__ __forceinline__ int sdot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// 8-lane horizontal tree of the reference's VEXTRACTF128 / VADDPS /
// VHADDPS / VHADDPS sequence: a_k = v_k + v_{k+4}; (a0 + a1) + (a2 + a3).
// Lanes k = 0..7 must be 8 consecutive lanes; lane k == 0 ends with the sum.
__device__ __forceinline__ float tree8(float v) {
    v = v + __shfl_xor(v, 4, 8);
    v = v + __shfl_xor(v, 1, 8);
    v = v + __shfl_xor(v, 2, 8);
    return v;
}

}  // namespace gllm
