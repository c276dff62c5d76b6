// Sticky error bits of the kernels (per GPU, per source file).
//
// Every bounded wait of the kernels (a correct run never reaches its bound) and every index
// that is clamped so that a broken invariant cannot read or write out of bounds reports it
// here: the kernel ORs a bit into an error word on the GPU. A correct call sets none, so a
// non-zero word means that some call gave up a wait or read a clamped row, i.e. returned
// wrong bits with rc 0. exkv_error_bits() gathers the words (and clears them) in stream
// order.
//
// Each source file that includes this header has its own word: a file-scope __device__
// variable, named only in device code (the kernels, and this file's fetch kernel, which
// the host launches through fetch_file_errors; host code never takes its address).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace exkv {

enum : uint32_t {
    kErrWait = 1u << 0,      // attention: a wait on another wavefront's LDS flag gave up
    kErrRawSlot = 1u << 1,   // attention / decode: a raw row's pool slot fell outside the pool
    kErrLookback = 1u << 2,  // encoder: the slot scan's look-back gave up on a predecessor
    kErrScanWs = 1u << 3,    // encoder: the scan workspace was inconsistent (more tickets than blocks)
    kErrWire = 1u << 4,      // wire unpack / pack: a raw row's pool slot fell outside the pool
};

static __device__ uint32_t file_error_word;

// Report from any lane (relaxed, device scope: the word is read after the stream's kernels
// have completed).
__device__ inline void report_error(uint32_t bits) {
    __hip_atomic_fetch_or(&file_error_word, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// out[0] = word (first) or out[0] | word; clear: the word is reset.
static __global__ void __launch_bounds__(64) error_fetch_kernel(uint32_t* out, int first, int clear) {
    if (threadIdx.x != 0) return;
    const uint32_t w = clear ? __hip_atomic_exchange(&file_error_word, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                             : __hip_atomic_load(&file_error_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    out[0] = first ? w : (out[0] | w);
}

static inline hipError_t fetch_file_errors(uint32_t* out, int first, int clear, hipStream_t stream) {
    hipLaunchKernelGGL(error_fetch_kernel, dim3(1), dim3(64), 0, stream, out, first, clear);
    return hipGetLastError();
}

// Slot of a raw row at rank `rank` of a page whose first raw slot is roff, clamped to the
// pool [0, raw_rows); bad is set when the clamp changed it. Host-callable, so that the CPU
// build can test it.
__host__ __device__ inline int64_t clamp_slot(int64_t slot, int64_t raw_rows, bool& bad) {
    bad = slot < 0 || slot >= raw_rows;
    return slot < 0 ? 0 : (slot >= raw_rows ? raw_rows - 1 : slot);
}

}  // namespace exkv
