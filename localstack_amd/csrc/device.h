// device.h - device helpers shared by the gfx950 kernels (kernels.hip, grouped.hip): fp16
// conversion, wavefront reductions over DPP, the Q8_0 / Q8_K activation quantizer and the Q4_K
// 6-bit scale / min unpacking.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>

#include "formats.h"
#include "kernels.h"

namespace lstk {
namespace {

constexpr int kWave = 64;

__device__ __forceinline__ float h2f(unsigned h) { return __half2float(__ushort_as_half((unsigned short) (h & 0xffffu))); }
__device__ __forceinline__ float round_f16(float x) { return __half2float(__float2half_rn(x)); }

// ------------------------------------------------------------------------------------------------
// wavefront reductions without LDS: DPP within 16-lane rows, readlane across rows
// ------------------------------------------------------------------------------------------------

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int) (u & 0xffffffffu), CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int) (u >> 32), CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(double, ((unsigned long long) (unsigned) hi << 32) | (unsigned) lo);
}
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ double readlane_d(double v, int l) {
    const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
    const unsigned lo = (unsigned) __builtin_amdgcn_readlane((int) (u & 0xffffffffu), l);
    const unsigned hi = (unsigned) __builtin_amdgcn_readlane((int) (u >> 32), l);
    return __builtin_bit_cast(double, ((unsigned long long) hi << 32) | lo);
}

// Sum over the 64 lanes as a pairwise tree: lanes l and l^1, then quads, octets, halves of rows,
// rows (0+1, 2+3) and the two row pairs. IEEE addition is commutative, so every lane of a level
// holds the same partial; the oracle evaluates the same tree. Result uniform.
__device__ __forceinline__ float wave_sum_tree(float v) {
    v = v + dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v = v + dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v = v + dpp_f<0x141>(v);  // row_half_mirror: the other quad of the octet
    v = v + dpp_f<0x140>(v);  // row_mirror: the other octet of the row
    return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}

__device__ __forceinline__ double wave_sum_d(double v) {
    v = v + dpp_d<0xB1>(v);
    v = v + dpp_d<0x4E>(v);
    v = v + dpp_d<0x141>(v);
    v = v + dpp_d<0x140>(v);
    return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

// ------------------------------------------------------------------------------------------------
// activation quantization (ggml's quantize_row_q8_0 x86 path / quantize_row_q8_K_ref)
// ------------------------------------------------------------------------------------------------

// Quantizes x[0..n) (n % 256 == 0) with all threads of the block, 8 values per thread per pass.
// Q8_0 (QT 8): d = amax/127 stored as fp16, q = rne(x * 127/amax), groups of 4 threads per block.
// Q8_K (QT 12): max = the signed value of the first largest |x| of the 256, iscale = -127/max,
// q = min(127, rne(iscale x)), d = 1/iscale; groups of 32 threads; bs = sums of 32-value groups.
// Every thread runs the shuffles; threads past the end contribute zeros and write nothing.
template <int QT>
__device__ __forceinline__ void quantize_row(const float *__restrict__ x, int n, int8_t *qs, float *d, int32_t *bs) {
    for (int base = 0; base < n; base += blockDim.x * 8) {
        const int i0 = base + threadIdx.x * 8;
        const bool on = i0 < n;
        float v[8];
        if (on) {
            const float4 a = *reinterpret_cast<const float4 *>(x + i0);
            const float4 b = *reinterpret_cast<const float4 *>(x + i0 + 4);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = 0.0f;
        }
        int q[8];
        float dd;
        if (QT == kTypeQ8_0) {
            float amax = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(v[j]));
            amax = fmaxf(amax, dpp_f<0xB1>(amax)); // the 4 threads of a 32-value block
            amax = fmaxf(amax, dpp_f<0x4E>(amax));
            dd = round_f16(__fdiv_rn(amax, 127.0f));
            const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) q[j] = (int) rintf(v[j] * id);
        } else {
            // (|x|, x, index) of the first largest |x|: 32 threads per 256-value block
            float amax = 0.0f, mx = 0.0f;
            int idx = INT_MAX;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float ax = fabsf(v[j]);
                if (ax > amax) {
                    amax = ax;
                    mx = v[j];
                    idx = i0 + j;
                }
            }
            auto take = [&](float oa, float om, int oi) {
                if (oa > amax || (oa == amax && oi < idx)) {
                    amax = oa;
                    mx = om;
                    idx = oi;
                }
            };
            take(dpp_f<0xB1>(amax), dpp_f<0xB1>(mx), __builtin_amdgcn_update_dpp(0, idx, 0xB1, 0xF, 0xF, false));
            take(dpp_f<0x4E>(amax), dpp_f<0x4E>(mx), __builtin_amdgcn_update_dpp(0, idx, 0x4E, 0xF, 0xF, false));
            take(dpp_f<0x141>(amax), dpp_f<0x141>(mx), __builtin_amdgcn_update_dpp(0, idx, 0x141, 0xF, 0xF, false));
            take(dpp_f<0x140>(amax), dpp_f<0x140>(mx), __builtin_amdgcn_update_dpp(0, idx, 0x140, 0xF, 0xF, false));
            // rows 0+1 form the block of lanes 0-31, rows 2+3 the block of lanes 32-63
            const int lane = threadIdx.x % kWave;
            const int r0 = lane < 32 ? 0 : 32;
            const float a0 = readlane_f(amax, 0), a1 = readlane_f(amax, 16), a2 = readlane_f(amax, 32), a3 = readlane_f(amax, 48);
            const float m0 = readlane_f(mx, 0), m1 = readlane_f(mx, 16), m2 = readlane_f(mx, 32), m3 = readlane_f(mx, 48);
            const int x0 = __builtin_amdgcn_readlane(idx, 0), x1 = __builtin_amdgcn_readlane(idx, 16);
            const int x2 = __builtin_amdgcn_readlane(idx, 32), x3 = __builtin_amdgcn_readlane(idx, 48);
            amax = r0 ? a2 : a0;
            mx = r0 ? m2 : m0;
            idx = r0 ? x2 : x0;
            take(r0 ? a3 : a1, r0 ? m3 : m1, r0 ? x3 : x1);
            if (amax == 0.0f) {
                dd = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; j++) q[j] = 0;
            } else {
                const float iscale = __fdiv_rn(-127.0f, mx);
#pragma unroll
                for (int j = 0; j < 8; j++) q[j] = min(127, (int) rintf(iscale * v[j]));
                dd = __fdiv_rn(1.0f, iscale);
            }
        }
        int s = 0;
#pragma unroll
        for (int j = 0; j < 8; j++) s += q[j];
        s += __builtin_amdgcn_update_dpp(0, s, 0xB1, 0xF, 0xF, false);
        s += __builtin_amdgcn_update_dpp(0, s, 0x4E, 0xF, 0xF, false);
        if (on) {
            uint2 packed;
            packed.x = (unsigned) (q[0] & 0xff) | ((unsigned) (q[1] & 0xff) << 8) | ((unsigned) (q[2] & 0xff) << 16) |
                       ((unsigned) (q[3] & 0xff) << 24);
            packed.y = (unsigned) (q[4] & 0xff) | ((unsigned) (q[5] & 0xff) << 8) | ((unsigned) (q[6] & 0xff) << 16) |
                       ((unsigned) (q[7] & 0xff) << 24);
            *reinterpret_cast<uint2 *>(qs + i0) = packed;
            if ((threadIdx.x & 3) == 0) {
                d[i0 / 32] = dd;
                bs[i0 / 32] = s;
            }
        }
    }
}

// get_scale_min_k4 on the 12 scale bytes held in three dwords.
template <int J>
__device__ __forceinline__ void scale_min_k4(unsigned s0, unsigned s1, unsigned s2, int &sc, int &m) {
    auto byte = [&](int i) -> int {
        const unsigned word = i < 4 ? s0 : (i < 8 ? s1 : s2);
        return (int) ((word >> (8 * (i & 3))) & 0xffu);
    };
    if (J < 4) {
        sc = byte(J) & 63;
        m = byte(J + 4) & 63;
    } else {
        sc = (byte(J + 4) & 0xF) | ((byte(J - 4) >> 6) << 4);
        m = (byte(J + 4) >> 4) | ((byte(J) >> 6) << 4);
    }
}

// A launch on `st`; with `tm` set, the launch records its own start / stop timestamps.
template <typename K, typename... A>
hipError_t launch(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t st, const LaunchTiming *tm, A... args) {
    if (tm && tm->start) hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t) lds, st, tm->start, tm->stop, 0, args...);
    else hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
    return hipGetLastError();
}

}  // namespace
}  // namespace lstk
