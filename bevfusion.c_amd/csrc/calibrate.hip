// Machine calibration kernels for the roofline discussion: launch cost, the
// sustained bf16 MFMA rate of the two instruction shapes the contractions
// use, the fp16 MFMA rate when the operands come from LDS as in the GEMM
// cores (with random or constant operand values), LDS read bandwidth and
// device-memory copy bandwidth.  Each kernel
// does a known amount of work; the caller times it with HIP events and turns
// the count into a rate.  Nothing here is on the product path.
#include "bfhip_profile.h"
#include "hip_common.h"

#include <climits>

using namespace bfhip;

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

__global__ void calib_empty_kernel() {}

// kChains independent accumulator chains per wave, so the MFMA pipeline is
// never waiting on its own result; operands come from registers seeded by the
// lane id.  One flag-guarded store keeps the work live.
constexpr int kChains = 8;

__global__ __launch_bounds__(256) void calib_mfma16_kernel(int iters, float *sink, int flag) {
    const int lane = threadIdx.x & 63;
    bf16x8 a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[e] = to_bf16(0.001f * (lane + e));
        b[e] = to_bf16(0.002f * (lane - e));
    }
    f32x4 acc[kChains];
#pragma unroll
    for (int c = 0; c < kChains; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int i = 0; i < iters; ++i)
#pragma unroll
        for (int c = 0; c < kChains; ++c) acc[c] = mfma16(a, b, acc[c]);
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < kChains; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
    if (flag) sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

__global__ __launch_bounds__(256) void calib_mfma32_kernel(int iters, float *sink, int flag) {
    const int lane = threadIdx.x & 63;
    bf16x8 a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[e] = to_bf16(0.001f * (lane + e));
        b[e] = to_bf16(0.002f * (lane - e));
    }
    constexpr int kC32 = kChains;
    f32x16 acc[kC32];
#pragma unroll
    for (int c = 0; c < kC32; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[c][r] = 0.f;
    for (int i = 0; i < iters; ++i)
#pragma unroll
        for (int c = 0; c < kC32; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < kC32; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[c][r];
    if (flag) sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Every lane reads 16 bytes per read from a 64 KiB LDS array, consecutive
// lanes consecutive 16-byte slots (conflict-free); each step issues kLdsBurst
// independent reads before using any, so the LDS pipe (not its latency) is
// the limit.  The empty asm keeps every step's reads inside the loop.
constexpr int kLdsBurst = 8;

__global__ __launch_bounds__(256) void calib_lds_kernel(int iters, float *sink, int flag) {
    constexpr int kSlots = 4096;  // 16-byte slots: 64 KiB
    __shared__ __attribute__((aligned(16))) float4 buf[kSlots];
    const int t = threadIdx.x;
    for (int i = t; i < kSlots; i += blockDim.x) buf[i] = make_float4((float)i, 1.f, 2.f, 3.f);
    __syncthreads();
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int i = 0; i < iters; i += kLdsBurst) {
        float4 v[kLdsBurst];
#pragma unroll
        for (int j = 0; j < kLdsBurst; ++j) v[j] = buf[(t + (i + j) * 256) & (kSlots - 1)];
#pragma unroll
        for (int j = 0; j < kLdsBurst; ++j) {
            acc.x += v[j].x; acc.y += v[j].y; acc.z += v[j].z; acc.w += v[j].w;
        }
        asm volatile("" ::: "memory");
    }
    if (flag) sink[blockIdx.x * blockDim.x + t] = acc.x + acc.y + acc.z + acc.w;
}

// MFMA fed from LDS the way the GEMM main loops feed it: WAVES waves, each
// owning an (FM*16) x (FN*16) tile, read their A and B fragments for every
// 32-deep step from a 64-deep swizzled LDS tile (conflict-free
// ds_read_b128), then issue FM*FN v_mfma_f32_16x16x32_f16.  RANDOM fills the
// tiles with hashed fp16 values in [-1, 1); otherwise with a few small
// integers.  The matrix cores draw more power on toggling operand bits, so
// the random variant is the rate real activations and weights can sustain.
// Per workgroup and iteration: 2 * FM * FN MFMAs and 2 * (FM + FN) KiB of
// LDS reads per wave.
template <int FM, int FN, int WAVES, bool RANDOM>
__global__ __launch_bounds__(WAVES * 64) void calib_lds_mfma_kernel(int iters, float *sink, int flag) {
    constexpr int kRows = 128, kBK = 64;
    __shared__ __attribute__((aligned(1024))) bf16 sA[kRows * kBK], sB[kRows * kBK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < kRows * kBK; i += WAVES * 64) {
        if (RANDOM) {
            uint32_t h = (uint32_t)i * 2654435761u + blockIdx.x * 97u;
            h ^= h >> 13;
            h *= 0x5bd1e995u;
            h ^= h >> 15;
            sA[i] = to_half((float)(h & 0xffffu) * (1.0f / 32768.0f) - 1.0f);
            sB[i] = to_half((float)(h >> 16) * (1.0f / 32768.0f) - 1.0f);
        } else {
            sA[i] = to_half((float)(i & 7));
            sB[i] = to_half((float)(i & 3));
        }
    }
    __syncthreads();
    const int swz = lane & 7;  // 64-deep tile swizzle of the LDS-DMA core
    const int a_row = ((wave * 16) % (kRows - FM * 16 + 16) + (lane & 15)) * kBK;
    const int b_row = ((wave * 32) % (kRows - FN * 16 + 16) + (lane & 15)) * kBK;
    int koff[2];
    for (int st = 0; st < 2; ++st) koff[st] = 8 * ((4 * st + (lane >> 4)) ^ swz);
    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            bf16x8 af[FM], bfr[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) af[i] = *reinterpret_cast<const bf16x8 *>(sA + a_row + i * 16 * kBK + koff[st]);
#pragma unroll
            for (int j = 0; j < FN; ++j) bfr[j] = *reinterpret_cast<const bf16x8 *>(sB + b_row + j * 16 * kBK + koff[st]);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = mfma16_f16(af[i], bfr[j], acc[i][j]);
        }
        asm volatile("" ::: "memory");
    }
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) t += acc[i][j][0];
    if (flag) sink[blockIdx.x * blockDim.x + tid] = t;
}

// y = x over n float4 (grid-stride): 2 * 16 * n bytes of device memory traffic.
__global__ __launch_bounds__(256) void calib_copy_kernel(const float4 *__restrict__ x,
                                                         float4 *__restrict__ y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        y[i] = x[i];
}

}  // namespace

extern "C" int bfhip_calibrate(int kind, int grid, int iters, const void *src, void *dst,
                               size_t bytes, void *stream_value, char *error, size_t cap) {
    hipStream_t s = reinterpret_cast<hipStream_t>(stream_value);
    if (grid <= 0 || iters < 0 || (kind == BFHIP_CALIB_LDS && iters % kLdsBurst))
        return fail(error, cap, "invalid calibration launch");
    float *sink = static_cast<float *>(dst);
    switch (kind) {
        case BFHIP_CALIB_EMPTY:
            hipLaunchKernelGGL(calib_empty_kernel, dim3(grid), dim3(64), 0, s);
            break;
        case BFHIP_CALIB_MFMA16:
        case BFHIP_CALIB_MFMA32:
        case BFHIP_CALIB_LDS: {
            // The sink holds one float per thread; it is written only when it
            // is large enough (the flag is otherwise 0 and nothing is stored).
            const size_t need = (size_t)grid * 256 * sizeof(float);
            const int flag = sink && bytes >= need ? 1 : 0;
            if (kind == BFHIP_CALIB_MFMA16)
                hipLaunchKernelGGL(calib_mfma16_kernel, dim3(grid), dim3(256), 0, s, iters, sink, flag);
            else if (kind == BFHIP_CALIB_MFMA32)
                hipLaunchKernelGGL(calib_mfma32_kernel, dim3(grid), dim3(256), 0, s, iters, sink, flag);
            else
                hipLaunchKernelGGL(calib_lds_kernel, dim3(grid), dim3(256), 0, s, iters, sink, flag);
            break;
        }
        case BFHIP_CALIB_MFMA_LDS:
        case BFHIP_CALIB_MFMA_LDS_FLAT:
        case BFHIP_CALIB_MFMA_LDS_NARROW:
        case BFHIP_CALIB_MFMA_LDS_NARROW_FLAT: {
            const size_t need = (size_t)grid * 512 * sizeof(float);
            const int flag = sink && bytes >= need ? 1 : 0;
            if (kind == BFHIP_CALIB_MFMA_LDS)
                hipLaunchKernelGGL((calib_lds_mfma_kernel<4, 4, 8, true>), dim3(grid), dim3(512), 0, s,
                                   iters, sink, flag);
            else if (kind == BFHIP_CALIB_MFMA_LDS_FLAT)
                hipLaunchKernelGGL((calib_lds_mfma_kernel<4, 4, 8, false>), dim3(grid), dim3(512), 0, s,
                                   iters, sink, flag);
            else if (kind == BFHIP_CALIB_MFMA_LDS_NARROW)
                hipLaunchKernelGGL((calib_lds_mfma_kernel<2, 2, 8, true>), dim3(grid), dim3(512), 0, s,
                                   iters, sink, flag);
            else
                hipLaunchKernelGGL((calib_lds_mfma_kernel<2, 2, 8, false>), dim3(grid), dim3(512), 0, s,
                                   iters, sink, flag);
            break;
        }
        case BFHIP_CALIB_COPY:
            if (!src || !dst || bytes % 16 || ((uintptr_t)src & 15) || ((uintptr_t)dst & 15))
                return fail(error, cap, "calibration copy needs 16-byte aligned buffers");
            hipLaunchKernelGGL(calib_copy_kernel, dim3(grid), dim3(256), 0, s,
                               static_cast<const float4 *>(src), static_cast<float4 *>(dst), bytes / 16);
            break;
        default:
            return fail(error, cap, "unknown calibration kernel %d", kind);
    }
    return launch_ok(error, cap, "launch calibration kernel");
}
