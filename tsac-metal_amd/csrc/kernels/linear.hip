// W8A8 quantised linear: y = bf16(sum_b fma(dot_b, w_scale[b][n] * a_scale[m][b]) + bias[n]).
//
// The int8 dot of each 256-value block is exact in int32 (|dot| <= 256*128*128
// < 2^24), so any summation order inside a block gives the same integer; only
// the fp32 chain over blocks has a fixed order (ascending b, one fma each), as
// in src/scalar/packed_linear.cpp:16-27. Both paths below compute the exact
// block dots and then run that same chain, so GEMV and GEMM agree bit for bit
// with each other and with the reference.
//
// Weights live in HBM in "row tiles", laid out once at load time: 64 output rows
// x one 256-value block form a 16 KiB tile stored as [segment 0..15][row 0..63]
// [16 bytes], tiles ordered [N/64][K/256]. A wavefront load of one segment is
// then 1 KiB contiguous with lane l holding row l.
//
//  * GEMV (decode, M <= 8 columns): one workgroup per 64-row tile, one
//    wavefront per block; every lane accumulates its row's whole block dot with
//    v_dot4 against wave-uniform activations (no cross-lane reduction), then the
//    ordered chain runs per (row, column) from LDS.
//  * GEMM (encode, large M): persistent 256-thread workgroups over 128x128
//    output tiles, int8 MFMA 32x32x32 into int32 accumulators per 256-wide K
//    block, operands streamed through an LDS ring by direct global->LDS loads,
//    and the per-block fp32 fma epilogue into a second accumulator set.
#include "device_numeric.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <cstdint>
#include <cstring>

namespace tsac_hip
{
namespace
{
constexpr int tile_rows = 64;
constexpr int segments = 16; // 16-byte segments per 256-value block

__device__ __forceinline__ uint16_t finish(float sum, float bias, const uint16_t* residual,
                                           std::size_t index)
{
    const uint16_t y = float_to_bf16(sum + bias);
    if (residual)
    {
        return float_to_bf16(bf16_to_float(residual[index]) + bf16_to_float(y));
    }
    return y;
}

// Byte offset of segment `s` of block `b` in row tile `t` (row 0 of the tile).
__device__ __forceinline__ std::size_t tile_offset(int t, int b, int s, int blocks)
{
    return ((std::size_t(t) * blocks + b) * segments + s) * (tile_rows * 16);
}

// ------------------------------------------------------------------ GEMV

constexpr int gemv_waves = 4;

// A GEMV reads every weight byte once per launch, so weight loads carry the
// nontemporal hint: streamed lines do not displace reusable ones. Measured on
// 1 GiB of rotating K = 1024 weights this raises the read rate from 70% to 80%
// of HBM peak; with cache-resident weights it changes nothing.
typedef unsigned int stream4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 stream_load(const int8_t* p)
{
    const stream4 v = __builtin_nontemporal_load(reinterpret_cast<const stream4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
constexpr int gemv_max_columns = 8;

template <int M>
__global__ __launch_bounds__(gemv_waves * wave) void gemv_kernel(
    const int8_t* __restrict__ weights, const float* __restrict__ weight_scales,
    const float* __restrict__ bias, int N, int K, const int8_t* __restrict__ q,
    const float* __restrict__ activation_scales, uint16_t* y, const uint16_t* residual)
{
    extern __shared__ int block_dots[]; // [blocks][M][64]
    const int blocks = K / 256;
    const int tile = blockIdx.x;
    const int lane = threadIdx.x % wave;
    const int warp = __builtin_amdgcn_readfirstlane(threadIdx.x / wave);
    for (int b = warp; b < blocks; b += gemv_waves)
    {
        uint4 w[segments];
        const int8_t* base = weights + tile_offset(tile, b, 0, blocks) + lane * 16;
#pragma unroll
        for (int s = 0; s < segments; ++s)
        {
            w[s] = stream_load(base + s * tile_rows * 16);
        }
        int dot[M];
#pragma unroll
        for (int m = 0; m < M; ++m)
        {
            dot[m] = 0;
            const uint4* a = reinterpret_cast<const uint4*>(q + std::size_t(m) * K + b * 256);
#pragma unroll
            for (int s = 0; s < segments; ++s)
            {
                const uint4 x = a[s];
                dot[m] = __builtin_amdgcn_sdot4(int(w[s].x), int(x.x), dot[m], false);
                dot[m] = __builtin_amdgcn_sdot4(int(w[s].y), int(x.y), dot[m], false);
                dot[m] = __builtin_amdgcn_sdot4(int(w[s].z), int(x.z), dot[m], false);
                dot[m] = __builtin_amdgcn_sdot4(int(w[s].w), int(x.w), dot[m], false);
            }
            block_dots[(b * M + m) * tile_rows + lane] = dot[m];
        }
    }
    __syncthreads();
    // Ordered chain per (row, column): ascending blocks, one fma each.
    for (int pair = threadIdx.x; pair < M * tile_rows; pair += blockDim.x)
    {
        const int m = pair / tile_rows, row = pair % tile_rows;
        const int n = tile * tile_rows + row;
        float sum = 0.0f;
        for (int b = 0; b < blocks; ++b)
        {
            const float scale = weight_scales[std::size_t(b) * N + n] * activation_scales[m * blocks + b];
            sum = __builtin_fmaf(float(block_dots[(b * M + m) * tile_rows + row]), scale, sum);
        }
        const std::size_t index = std::size_t(m) * N + n;
        y[index] = finish(sum, bias[n], residual, index);
    }
}

void launch_gemv(const DeviceLinear& w, const int8_t* q, const float* scales, std::size_t M,
                 uint16_t* y, const uint16_t* residual, hipStream_t stream)
{
    const unsigned grid = unsigned(w.N / tile_rows);
    const std::size_t lds = (w.K / 256) * M * tile_rows * sizeof(int);
    const int N = int(w.N), K = int(w.K);
#define TSAC_GEMV(MM)                                                                              \
    case MM:                                                                                       \
        gemv_kernel<MM><<<grid, gemv_waves * wave, lds, stream>>>(w.values, w.scales, w.bias, N, K, \
                                                                  q, scales, y, residual);        \
        break;
    switch (M)
    {
        TSAC_GEMV(1)
        TSAC_GEMV(2)
        TSAC_GEMV(3)
        TSAC_GEMV(4)
        TSAC_GEMV(5)
        TSAC_GEMV(6)
        TSAC_GEMV(7)
        TSAC_GEMV(8)
    default:
        throw Error("gemv: column count out of range");
    }
#undef TSAC_GEMV
}

// ------------------------------------------------------------------ small M (MFMA)
//
// 8 < M <= 64 row-major rows and K <= 2048: one workgroup per 32 output columns
// and 32-row group, one wave per 256-value block. A wave loads its block's
// 32 x 256 weights from the row tile straight into registers in the MFMA's
// operand order (one 512-byte run per half-wave and 32-value k-slice) and its
// rows' block activations the same way, runs the block's exact int32 dots as
// 8 MFMAs (32 x 32 x 32), and leaves them in LDS; the ordered chain then runs
// per (row, column) as in the GEMV, with the scales staged in LDS while the
// operands arrive. No row is padded to a large tile, and the launch has
// N / 32 x ceil(M / 32) workgroups (measured: one workgroup per 32 columns for
// both row groups took 7.9 us at M = 64, K = 1024, N = 1024; split by row
// group, 5.5 us).

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int small_max_rows = 64;      // rows the automatic path always gives this kernel
constexpr int small_launch_max_rows = 1024; // rows one launch accepts
constexpr int small_max_blocks = 8;
constexpr int small_columns = 32;
constexpr int small_rows = 32;        // rows of a workgroup
constexpr int small_stride = small_columns + 1; // LDS row stride of the dots, conflict-free writes

__device__ __forceinline__ v4i load_fragment(const int8_t* p)
{
    return *reinterpret_cast<const v4i*>(p);
}

__global__ __launch_bounds__(small_max_blocks * wave) void small_gemm_kernel(
    const int8_t* __restrict__ weights, const float* __restrict__ weight_scales,
    const float* __restrict__ bias, int N, int K, const int8_t* __restrict__ q,
    const float* __restrict__ activation_scales, int M, uint16_t* y, const uint16_t* residual)
{
    __shared__ int dots[small_max_blocks * small_rows * small_stride]; // [block][row][column]
    __shared__ float ws[small_max_blocks * small_columns];              // [block][column]
    __shared__ float as[small_rows * small_max_blocks];                 // [row][block]
    __shared__ float bs[small_columns];
    const int blocks = K / 256;
    const int tile = blockIdx.x / 2, half = blockIdx.x % 2; // 32 of the 64 rows of a weight row tile
    const int n0 = blockIdx.x * small_columns, m0 = blockIdx.y * small_rows;
    const int rows = min(small_rows, M - m0);
    const int lane = threadIdx.x % wave;
    const int b = __builtin_amdgcn_readfirstlane(threadIdx.x / wave); // one wave per block
    // Operands first. A: lane l holds weight row l % 32 of this half, k-slice
    // values 16 (l / 32) .. +15; the 16-byte segments of a row tile are 1 KiB
    // apart, two per 32-value slice. B: lane l holds activation row m0 + l % 32
    // (the last row stands in for rows past M, whose results are not read),
    // the same values.
    const int8_t* w = weights + tile_offset(tile, b, lane / 32, blocks) + (half * 32 + lane % 32) * 16;
    const int8_t* x = q + std::size_t(m0 + min(lane % 32, rows - 1)) * K + b * 256 + (lane / 32) * 16;
    v4i a[8], u[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
    {
        a[j] = load_fragment(w + 2 * j * tile_rows * 16);
        u[j] = load_fragment(x + 32 * j);
    }
    for (int i = threadIdx.x; i < blocks * small_columns; i += blockDim.x)
    {
        ws[i] = weight_scales[std::size_t(i / small_columns) * N + n0 + i % small_columns];
    }
    for (int i = threadIdx.x; i < rows * blocks; i += blockDim.x)
    {
        as[i] = activation_scales[std::size_t(m0) * blocks + i];
    }
    if (threadIdx.x < small_columns)
    {
        bs[threadIdx.x] = bias[n0 + threadIdx.x];
    }
    const v16i zero = {};
    v16i acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[0], u[0], zero, 0, 0, 0);
#pragma unroll
    for (int j = 1; j < 8; ++j)
    {
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[j], u[j], acc, 0, 0, 0);
    }
    // Lane l, register r: row l % 32, column 8 (r / 4) + 4 (l / 32) + r % 4.
    int* d = dots + (b * small_rows + lane % 32) * small_stride + 4 * (lane / 32);
#pragma unroll
    for (int r = 0; r < 16; ++r)
    {
        d[8 * (r / 4) + r % 4] = acc[r];
    }
    __syncthreads();
    // Ordered chain per (row, column): ascending blocks, one fma each.
    for (int i = threadIdx.x; i < rows * small_columns; i += blockDim.x)
    {
        const int m = i / small_columns, c = i % small_columns;
        float sum = 0.0f;
        for (int k = 0; k < blocks; ++k)
        {
            const float scale = ws[k * small_columns + c] * as[m * blocks + k];
            sum = __builtin_fmaf(float(dots[(k * small_rows + m) * small_stride + c]), scale, sum);
        }
        const std::size_t index = std::size_t(m0 + m) * N + n0 + c;
        y[index] = finish(sum, bs[c], residual, index);
    }
}

void launch_small_gemm(const DeviceLinear& w, const int8_t* q, const float* scales, std::size_t M, uint16_t* y,
                       const uint16_t* residual, hipStream_t stream)
{
    require(M >= 1 && M <= std::size_t(small_launch_max_rows) && w.K <= std::size_t(small_max_blocks) * 256,
            "small-M GEMM: at most 1024 rows and K <= 2048");
    const dim3 grid(unsigned(w.N / small_columns), unsigned((M + small_rows - 1) / small_rows));
    const unsigned threads = unsigned(w.K / 256) * wave;
    small_gemm_kernel<<<grid, threads, 0, stream>>>(w.values, w.scales, w.bias, int(w.N), int(w.K), q, scales,
                                                    int(M), y, residual);
}

// ------------------------------------------------------------------ GEMM (MFMA)
//
// Persistent workgroups (two per CU) walk 128 x 128 output tiles. The tiles of
// each XCD are one contiguous run in (row panel, column tile) order, so a
// 128-row activation panel is fetched from HBM once and then reused from that
// XCD's L2 by all column tiles. Operands stream through an LDS ring filled by
// direct global->LDS loads (global_load_lds_dwordx4) Ring-1 stages ahead of the
// MFMAs. The stream runs on across tile boundaries: a workgroup's tiles form one
// sequence of stages, so the next tile's first stages load while the current
// tile finishes, and its outputs are stored from registers with no barrier.
//
// The MFMA's first operand is the weight tile and its second the activations:
// lane l, register r of a 32 x 32 result holds column n = 8*(r/4) + 4*(l/32) + r%4
// of row m = l%32, so each lane owns runs of four consecutive outputs of a row.

namespace gemm
{
constexpr int tile_n = 128, tile_m = int(gemm_tile_rows);
constexpr int scale_bytes = 4 * (tile_n + tile_m); // ws[128], then as[128]
constexpr int bias_bytes = 4 * tile_n;
constexpr int threads = 256;
constexpr int xcds = 8;

// StageK bytes of K per pipeline stage, Ring LDS stage slots, PerCU resident
// workgroups per CU; Preload reads a stage's operand fragments from LDS before
// its MFMAs (more registers, fewer exposed LDS latencies).
template <int StageK, int Ring, int PerCU, bool Preload> struct Config
{
    static_assert(StageK == 64 || StageK == 128, "stage depth");
    static_assert(Ring >= 2, "ring depth");
    static constexpr int stage_k = StageK, ring = Ring, per_cu = PerCU;
    static constexpr bool preload = Preload;
    static constexpr int slices = StageK / 32; // 32-byte MFMA k-slices per stage
    static constexpr int copies = StageK / 16; // 1 KiB operand copies per wave per stage
    static constexpr int stages_per_block = 256 / StageK;
    // Block b's scales are copied with its first stage, Ring-1 stages ahead,
    // and read after its last stage: the copies of the blocks issued in
    // between need slots of their own.
    static constexpr int scale_slots = (Ring - 2) / stages_per_block + 2;
    static constexpr int weight_bytes = tile_n * StageK; // 2 row tiles x StageK/16 segments
    static constexpr int stage_bytes = weight_bytes + tile_m * StageK; // + 4 row groups x slices
    // A tile's bias arrives Ring-1 stages before its first stage, while the
    // previous tile's epilogue may still read that tile's bias: two slots.
    static constexpr int lds_bytes = Ring * stage_bytes + scale_slots * scale_bytes + 2 * bias_bytes;
};
using Default = Config<128, 2, 2, true>;
// K <= 512: three workgroups per CU on 64-deep stages, measured 2-5% faster on
// the M = 30,960 K = 512 shapes (and slower at K = 2048).
using ShortK = Config<64, 2, 3, true>;
} // namespace gemm

// One wavefront copies 64 x 16 bytes (or 64 x 4) from per-lane global addresses
// to LDS at `lds` + 16*lane (4*lane); `lds` is wave-uniform. Issued as inline
// assembly: the compiler's wait insertion treats the builtin form as aliasing
// every later LDS read and drains all loads in flight before each one, which
// would serialise the ring. Completion is tracked explicitly with
// wait_vector_memory, and the "memory" clobber keeps LDS accesses in order.
__device__ __forceinline__ uint32_t lds_address(const void* p)
{
    return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}
// M0 is reserved, so clang warns about naming it as a clobber; these kernels
// use M0 for nothing else, and naming it keeps the compiler from assuming
// that a value it put there survives.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void copy_to_lds16(const void* src, const void* lds)
{
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_address(lds))
                 : "memory", "m0");
}
__device__ __forceinline__ void copy_to_lds4(const void* src, const void* lds)
{
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(lds_address(lds))
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt vmcnt(N) lgkmcnt(0): at most N of this wave's vector memory
// operations still outstanding (they complete in issue order), LDS reads done.
template <int N> __device__ __forceinline__ void wait_vector_memory()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}
// The same for a wave-uniform count known only at run time (binary search
// over the immediates; counts above 63 wait for 63, which is stricter).
template <int Lo, int Hi> __device__ __forceinline__ void wait_vector_memory_at_most(int n)
{
    if constexpr (Lo == Hi)
    {
        wait_vector_memory<Lo>();
    }
    else
    {
        constexpr int mid = (Lo + Hi + 1) / 2;
        if (n >= mid)
        {
            wait_vector_memory_at_most<mid, Hi>(n);
        }
        else
        {
            wait_vector_memory_at_most<Lo, mid - 1>(n);
        }
    }
}

// Workgroup barrier without the vmcnt(0) that __syncthreads() implies, which
// would drain the loads in flight. It does wait for this wave's own LDS
// accesses (lgkmcnt(0)), so LDS writes before it are visible to every wave
// after it. The empty asm statements keep the compiler from moving memory
// accesses across it.
__device__ __forceinline__ void ring_barrier()
{
    asm volatile("" ::: "memory");
    wait_vector_memory<63>(); // vmcnt(63) waits for nothing; lgkmcnt(0) does
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Outputs leave straight from the accumulator registers. Lane l holds columns
// 8g + 4(l/32) + 0..3 of row l%32 for register group g; one permlane32 swap per
// pair of groups (g, g+1) gives the low half-wave columns 8g..8g+7 and the high
// half-wave columns 8(g+1)..8(g+1)+7, so every lane stores 16 bytes.
typedef unsigned int out4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi)
{
    return uint32_t(float_to_bf16(lo)) | (uint32_t(float_to_bf16(hi)) << 16);
}
__device__ __forceinline__ uint32_t add_bf16_pair(uint32_t r, uint32_t v)
{
    const uint32_t lo = float_to_bf16(bf16_to_float(uint16_t(r & 0xffff)) + bf16_to_float(uint16_t(v & 0xffff)));
    const uint32_t hi = float_to_bf16(bf16_to_float(uint16_t(r >> 16)) + bf16_to_float(uint16_t(v >> 16)));
    return lo | (hi << 16);
}
// Raw buffer resource over `bytes` bytes (gfx9 dword3): accesses past the end
// are dropped (stores) or read zero (loads).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t byte_buffer(const void* base, int bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

template <bool Tiles, class Cfg>
__global__ __launch_bounds__(gemm::threads, Cfg::per_cu) void gemm_kernel(
    const int8_t* __restrict__ weights, const float* __restrict__ weight_scales,
    const float* __restrict__ bias, int N, int K, const int8_t* __restrict__ q,
    const float* __restrict__ activation_scales, int M, int padded_rows, uint16_t* y,
    const uint16_t* residual)
{
    using namespace gemm;
    constexpr int ring = Cfg::ring, slices = Cfg::slices, copies = Cfg::copies;
    constexpr int spb = Cfg::stages_per_block, weight_bytes = Cfg::weight_bytes, stage_bytes = Cfg::stage_bytes;
    constexpr int scale_slots = Cfg::scale_slots;
    constexpr int stores = 8; // 16-byte output stores per wave per tile
    __shared__ __attribute__((aligned(1024))) int8_t lds[Cfg::lds_bytes];
    const int lane = threadIdx.x % wave;
    const int warp = __builtin_amdgcn_readfirstlane(threadIdx.x / wave);
    const int wn = warp % 2, wm = warp / 2;
    const int blocks = K / 256, stages = K / Cfg::stage_k;
    const int row_tiles = N / tile_rows;
    const int n_tiles = (N + tile_n - 1) / tile_n;
    const int total = n_tiles * ((M + tile_m - 1) / tile_m);
    const int per_xcd = gridDim.x / xcds;
    const int xcd = blockIdx.x % xcds;
    const int end = int(int64_t(total) * (xcd + 1) / xcds);
    const int first = int(int64_t(total) * xcd / xcds) + int(blockIdx.x / xcds);
    const int my_tiles = first < end ? (end - first + per_xcd - 1) / per_xcd : 0;
    const int total_stages = my_tiles * stages;
    float* const scale_ring = reinterpret_cast<float*>(lds + ring * stage_bytes);
    float* const bias_ring = scale_ring + scale_slots * (scale_bytes / 4);
    const int output_bytes = M * N * 2;
    const __amdgpu_buffer_rsrc_t output = byte_buffer(y, output_bytes);
    const __amdgpu_buffer_rsrc_t residual_in = byte_buffer(residual, output_bytes);

    // Global stage G = k * stages + s is stage s of this workgroup's k-th tile:
    // `copies` 1 KiB operand copies per wave (waves 0-1 weights, 2-3
    // activations), at a block start one 256-byte scale copy per wave, and at
    // a tile start the tile's bias (waves 0-1, into one of two bias slots).
    const auto issue = [&](int G)
    {
        const int k = G / stages, s = G - k * stages;
        const int tile = first + k * per_xcd;
        const int m_tile = tile / n_tiles, n_tile = tile % n_tiles;
        const int b = s / spb;
        int8_t* slot = lds + (G % ring) * stage_bytes;
        if (warp < 2)
        {
            const int t = min(n_tile * 2 + warp, row_tiles - 1);
            const int8_t* src = weights + tile_offset(t, b, (s % spb) * copies, blocks) + lane * 16;
#pragma unroll
            for (int i = 0; i < copies; ++i)
            {
                copy_to_lds16(src + i * tile_rows * 16, slot + (warp * copies + i) * 1024);
            }
        }
        else
        {
#pragma unroll
            for (int i = 0; i < copies; ++i)
            {
                const int c = (warp - 2) * copies + i, group = c / slices, slice = c % slices;
                const int8_t* src;
                if constexpr (Tiles)
                {
                    src = q + (std::size_t(m_tile * 4 + group) * (K / 32) + s * slices + slice) * 1024 + lane * 16;
                }
                else
                {
                    const int row = min(m_tile * tile_m + group * 32 + lane % 32, M - 1);
                    src = q + std::size_t(row) * K + s * Cfg::stage_k + slice * 32 + (lane / 32) * 16;
                }
                copy_to_lds16(src, slot + weight_bytes + (group * slices + slice) * 1024);
            }
        }
        if (s % spb == 0)
        {
            float* scales = scale_ring + ((G / spb) % scale_slots) * (scale_bytes / 4);
            const float* src;
            if (warp < 2)
            {
                const int n = min(n_tile * tile_n + warp * 64 + lane, N - 1);
                src = weight_scales + std::size_t(b) * N + n;
            }
            else
            {
                const int m = m_tile * tile_m + (warp - 2) * 64 + lane;
                src = Tiles ? activation_scales + std::size_t(b) * padded_rows + m
                            : activation_scales + std::size_t(min(m, M - 1)) * blocks + b;
            }
            copy_to_lds4(src, scales + warp * 64);
            if (s == 0 && warp < 2)
            {
                copy_to_lds4(bias + min(n_tile * tile_n + warp * 64 + lane, N - 1),
                             bias_ring + (k % 2) * tile_n + warp * 64);
            }
        }
    };
    // Vector memory operations this wave issues for global stage G.
    const auto count = [&](int G)
    {
        return copies + (G % spb == 0 ? 1 : 0) + (G % stages == 0 && warp < 2 ? 1 : 0);
    };

    v16i acc[2][2];
    float sum[2][2][16];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                sum[j][i][r] = 0.0f;
            }
    for (int G = 0; G < ring - 1 && G < total_stages; ++G)
    {
        issue(G);
    }
    // One stage of MFMAs; the first stage of a block starts its accumulators
    // from zero (the MFMA's C operand), so nothing clears them in between.
    const auto stage = [&](int G, auto first_of_block)
    {
        // Stage G has landed once only the operations issued after it may be
        // outstanding: the copies of stages G+1 .. G+ring-2 and, at a tile's
        // first stage, the previous tile's output stores (issued after those
        // copies; every wave issues all of them, see the epilogue).
        const int last = min(G + ring - 2, total_stages - 1);
        int younger = G % stages == 0 && G > 0 ? stores : 0;
        for (int g = G + 1; g <= last; ++g)
        {
            younger += count(g);
        }
        wait_vector_memory_at_most<0, 63>(younger);
        ring_barrier();
        if (G + ring - 1 < total_stages)
        {
            issue(G + ring - 1);
        }
        const int8_t* slot = lds + (G % ring) * stage_bytes;
        const auto fragment_w = [&](int slice, int j)
        {
            return *reinterpret_cast<const v4i*>(slot + (wn * copies + 2 * slice + lane / 32) * 1024 +
                                                 (j * 32 + lane % 32) * 16);
        };
        const auto fragment_x = [&](int slice, int i)
        {
            return *reinterpret_cast<const v4i*>(slot + weight_bytes + ((wm * 2 + i) * slices + slice) * 1024 +
                                                 lane * 16);
        };
        constexpr bool from_zero = decltype(first_of_block)::value;
        const v16i zero = {};
        if constexpr (Cfg::preload)
        {
            v4i a[slices][2], x[slices][2];
#pragma unroll
            for (int slice = 0; slice < slices; ++slice)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                {
                    a[slice][j] = fragment_w(slice, j);
                    x[slice][j] = fragment_x(slice, j);
                }
#pragma unroll
            for (int slice = 0; slice < slices; ++slice)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int i = 0; i < 2; ++i)
                    {
                        acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                            a[slice][j], x[slice][i], from_zero && slice == 0 ? zero : acc[j][i], 0, 0, 0);
                    }
        }
        else
        {
#pragma unroll
            for (int slice = 0; slice < slices; ++slice)
            {
                const v4i a[2] = {fragment_w(slice, 0), fragment_w(slice, 1)};
                const v4i x[2] = {fragment_x(slice, 0), fragment_x(slice, 1)};
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int i = 0; i < 2; ++i)
                    {
                        acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                            a[j], x[i], from_zero && slice == 0 ? zero : acc[j][i], 0, 0, 0);
                    }
            }
        }
    };

    for (int G = 0; G < total_stages; G += spb)
    {
        stage(G, std::true_type{});
#pragma unroll
        for (int t = 1; t < spb; ++t)
        {
            stage(G + t, std::false_type{});
        }
        // Block epilogue: one fp32 fma per output, blocks in ascending order.
        {
            const float* scales = scale_ring + ((G / spb) % scale_slots) * (scale_bytes / 4);
            float as[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
            {
                as[i] = scales[tile_n + wm * 64 + i * 32 + lane % 32];
            }
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int group = 0; group < 4; ++group)
                {
                    const float4 w4 = *reinterpret_cast<const float4*>(scales + wn * 64 + j * 32 + 8 * group +
                                                                       4 * (lane / 32));
                    const float ws[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e)
#pragma unroll
                        for (int i = 0; i < 2; ++i)
                        {
                            const int r = 4 * group + e;
                            sum[j][i][r] = __builtin_fmaf(float(acc[j][i][r]), ws[e] * as[i], sum[j][i][r]);
                        }
                }
        }
        if ((G + spb) % stages != 0)
        {
            continue;
        }
        // Tile epilogue: bias, BF16 (and the residual add), 16-byte stores from
        // registers. The next tile's first stages are already in flight.
        const int k = G / stages, tile = first + k * per_xcd;
        const int m_tile = tile / n_tiles, n_tile = tile % n_tiles;
        const float* bias_tile = bias_ring + (k % 2) * tile_n;
#pragma unroll
        for (int j = 0; j < 2; ++j)
        {
            float bn[4][4];
#pragma unroll
            for (int group = 0; group < 4; ++group)
            {
                const float4 b4 = *reinterpret_cast<const float4*>(bias_tile + wn * 64 + j * 32 + 8 * group +
                                                                   4 * (lane / 32));
                bn[group][0] = b4.x, bn[group][1] = b4.y, bn[group][2] = b4.z, bn[group][3] = b4.w;
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
            {
                const int row = m_tile * tile_m + wm * 64 + i * 32 + lane % 32;
                const float(&v)[16] = sum[j][i];
#pragma unroll
                for (int pair = 0; pair < 2; ++pair)
                {
                    const int g0 = 2 * pair, g1 = 2 * pair + 1;
                    const uint32_t p0 = pack_bf16(v[4 * g0 + 0] + bn[g0][0], v[4 * g0 + 1] + bn[g0][1]);
                    const uint32_t p1 = pack_bf16(v[4 * g0 + 2] + bn[g0][2], v[4 * g0 + 3] + bn[g0][3]);
                    const uint32_t q0 = pack_bf16(v[4 * g1 + 0] + bn[g1][0], v[4 * g1 + 1] + bn[g1][1]);
                    const uint32_t q1 = pack_bf16(v[4 * g1 + 2] + bn[g1][2], v[4 * g1 + 3] + bn[g1][3]);
                    const auto s0 = __builtin_amdgcn_permlane32_swap(p0, q0, false, false);
                    const auto s1 = __builtin_amdgcn_permlane32_swap(p1, q1, false, false);
                    const int column = n_tile * tile_n + wn * 64 + j * 32 + 8 * (g0 + lane / 32);
                    // Outputs outside the matrix get an offset past the buffer's
                    // end: the range check drops the store, but it is still
                    // issued, so every wave issues exactly `stores` of them.
                    const uint32_t offset =
                        row < M && column < N ? uint32_t(row * N + column) * 2 : 0x80000000u;
                    out4 out = {uint32_t(s0[0]), uint32_t(s1[0]), uint32_t(s0[1]), uint32_t(s1[1])};
                    if (residual)
                    {
                        const out4 r4 = __builtin_amdgcn_raw_buffer_load_b128(residual_in, offset, 0, 0);
                        out = out4{add_bf16_pair(r4[0], out[0]), add_bf16_pair(r4[1], out[1]),
                                   add_bf16_pair(r4[2], out[2]), add_bf16_pair(r4[3], out[3])};
                    }
                    __builtin_amdgcn_raw_buffer_store_b128(out, output, offset, 0, 0);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                {
                    sum[j][i][r] = 0.0f;
                }
    }
}

int compute_units()
{
    static const int count = []
    {
        int device = 0, units = 0;
        check_hip(hipGetDevice(&device), "hipGetDevice");
        check_hip(hipDeviceGetAttribute(&units, hipDeviceAttributeMultiprocessorCount, device),
                  "hipDeviceGetAttribute");
        return units > 0 ? units : 1;
    }();
    return count;
}

template <class Cfg>
void launch_gemm_config(const DeviceLinear& w, const int8_t* q, const float* scales, std::size_t M, uint16_t* y,
                        const uint16_t* residual, Layout layout, hipStream_t stream)
{
    using namespace gemm;
    require(M < (std::size_t(1) << 30), "gemm: too many rows");
    require(reinterpret_cast<uintptr_t>(y) % 16 == 0 && reinterpret_cast<uintptr_t>(residual) % 16 == 0,
            "gemm: output and residual must be 16-byte aligned");
    // The kernel addresses outputs through a buffer resource with a 32-bit
    // byte range, so one launch covers at most `chunk` rows (a multiple of the
    // 128-row tile); larger matrices take several launches.
    static_assert(256 % Cfg::stage_k == 0, "whole blocks per stage");
    const std::size_t chunk = std::max<std::size_t>(((std::size_t(1) << 31) - 1) / (2 * w.N) / tile_m * tile_m, tile_m);
    require(chunk * w.N * 2 < (std::size_t(1) << 31), "gemm: output row too wide");
    const int padded = int(tile_padded_rows(M));
    const std::size_t blocks = w.K / 256;
    for (std::size_t row0 = 0; row0 < M; row0 += chunk)
    {
        const std::size_t rows = std::min(chunk, M - row0);
        const std::size_t n_tiles = (w.N + tile_n - 1) / tile_n, m_tiles = (rows + tile_m - 1) / tile_m;
        const std::size_t total = n_tiles * m_tiles;
        std::size_t grid = std::size_t(compute_units()) * Cfg::per_cu;
        grid = std::min(grid, (total + xcds - 1) / xcds * xcds);
        grid = std::max<std::size_t>(grid / xcds * xcds, xcds);
        uint16_t* out = y + row0 * w.N;
        const uint16_t* add = residual ? residual + row0 * w.N : nullptr;
        if (layout == Layout::tiles)
        {
            // Row groups of 32 are 32*K contiguous bytes; scales are [b][padded].
            gemm_kernel<true, Cfg><<<unsigned(grid), threads, 0, stream>>>(
                w.values, w.scales, w.bias, int(w.N), int(w.K), q + row0 * w.K, scales + row0, int(rows), padded,
                out, add);
        }
        else
        {
            gemm_kernel<false, Cfg><<<unsigned(grid), threads, 0, stream>>>(
                w.values, w.scales, w.bias, int(w.N), int(w.K), q + row0 * w.K, scales + row0 * blocks, int(rows),
                padded, out, add);
        }
    }
}

void launch_gemm(const DeviceLinear& w, const int8_t* q, const float* scales, std::size_t M, uint16_t* y,
                 const uint16_t* residual, Layout layout, hipStream_t stream)
{
    if (w.K <= 512)
    {
        launch_gemm_config<gemm::ShortK>(w, q, scales, M, y, residual, layout, stream);
    }
    else
    {
        launch_gemm_config<gemm::Default>(w, q, scales, M, y, residual, layout, stream);
    }
}
} // namespace

std::size_t small_gemm_max_rows()
{
    return small_max_rows;
}

bool small_gemm_chosen(std::size_t M, std::size_t N, std::size_t K)
{
    // Up to 64 rows always. Up to 1024 rows too when the GEMM's 128 x 128
    // tiles would occupy at most a quarter of the compute units: the small-M
    // kernel's 32 x 32 workgroups then fill the chip instead (K = 1024,
    // N = 1024, M = 1024: 8.9 us against 12.5 us for 64 GEMM tiles; at 256
    // tiles, M = 4096 or N = 4096, the GEMM is twice as fast).
    if (M <= gemv_max_columns || K > std::size_t(small_max_blocks) * 256)
    {
        return false;
    }
    const std::size_t gemm_tiles = (M + gemm::tile_m - 1) / gemm::tile_m * ((N + gemm::tile_n - 1) / gemm::tile_n);
    return M <= std::size_t(small_max_rows) ||
           (M <= std::size_t(small_launch_max_rows) && gemm_tiles * 4 <= std::size_t(compute_units()));
}

std::size_t gemv_max_rows()
{
    return gemv_max_columns;
}

void tile_weights(const int8_t* canonical, std::size_t K, std::size_t N, int8_t* tiled)
{
    require(K % 256 == 0 && N % tile_rows == 0, "weights: K must be a multiple of 256, N of 64");
    const std::size_t blocks = K / 256;
    for (std::size_t n = 0; n < N; ++n)
    {
        const std::size_t t = n / tile_rows, lane = n % tile_rows;
        for (std::size_t b = 0; b < blocks; ++b)
        {
            for (std::size_t s = 0; s < segments; ++s)
            {
                std::memcpy(tiled + ((t * blocks + b) * segments + s) * tile_rows * 16 + lane * 16,
                            canonical + n * K + b * 256 + s * 16, 16);
            }
        }
    }
}

void linear(const DeviceLinear& w, const int8_t* q, const float* scales, std::size_t M,
            uint16_t* y, const uint16_t* residual, LinearPath path, hipStream_t stream, Layout layout)
{
    require(w.K >= 256 && w.K % 256 == 0 && w.K <= 4096, "linear: K must be a multiple of 256 <= 4096");
    require(w.N > 0 && w.N % tile_rows == 0 && w.N < (std::size_t(1) << 30),
            "linear: N must be a multiple of 64");
    if (M == 0)
    {
        return;
    }
    if (path == LinearPath::automatic)
    {
        path = layout != Layout::rows           ? LinearPath::gemm
               : M <= gemv_max_columns          ? LinearPath::gemv
               : small_gemm_chosen(M, w.N, w.K) ? LinearPath::small
                                                : LinearPath::gemm;
    }
    if (path == LinearPath::gemv)
    {
        require(M <= gemv_max_columns, "gemv: at most 8 columns");
        require(layout == Layout::rows, "gemv: activations must be row-major");
        launch_gemv(w, q, scales, M, y, residual, stream);
    }
    else if (path == LinearPath::small)
    {
        require(layout == Layout::rows, "small-M GEMM: activations must be row-major");
        launch_small_gemm(w, q, scales, M, y, residual, stream);
    }
    else
    {
        launch_gemm(w, q, scales, M, y, residual, layout, stream);
    }
    check_hip(hipGetLastError(), "linear launch");
}
} // namespace tsac_hip
