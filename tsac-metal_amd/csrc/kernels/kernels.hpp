// Host-side launchers for the probability-model kernels. Every launcher checks
// the shapes its kernel's indexing assumes and throws tsac_hip::Error before
// launching anything that would not fit.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

namespace tsac_hip
{
struct Error : std::runtime_error
{
    using std::runtime_error::runtime_error;
};

inline void require(bool condition, const char* message)
{
    if (!condition)
    {
        throw Error(message);
    }
}

inline void check_hip(hipError_t status, const char* what)
{
    if (status != hipSuccess)
    {
        throw Error(std::string(what) + ": " + hipGetErrorString(status));
    }
}

// Error words written by kernels (plain stores of fixed values):
// word 0 = a BF8L, softmax or categorical input was not finite; word 1 = the
// range decoder failed; word 2 = a frame-step wait stalled (see frame.hpp).
constexpr uint32_t error_nonfinite = 1u;

// ---- quantisation (BF8L, src/scalar/probability.cpp:16-40) ------------------
enum class Prologue
{
    none,       // quantise the BF16 rows as they are
    layer_norm, // LayerNorm (gain, bias) first (src/common/probability.cpp:138-169)
    gelu,       // GELU first (src/common/probability.cpp:45-63)
};

// Storage of quantised activations.
//  rows:  q [rows][K] int8, scales [rows][K/256].
//  tiles: MFMA operand tiles for the GEMM. Rows are padded to
//         tile_padded_rows(rows) (a multiple of gemm_tile_rows); byte k of row m
//         is at ((m/32)*(K/32) + k/32)*1024 + ((m%32) + 32*((k/16)%2))*16 + k%16,
//         and scales are transposed: scales[b*padded + m]. Padding rows are never
//         written and only ever feed outputs that are not stored.
enum class Layout
{
    rows,
    tiles
};
constexpr std::size_t gemm_tile_rows = 128;
std::size_t tile_padded_rows(std::size_t rows);

// x: [rows][K] BF16 -> q, scales in `layout` (fp32 scales are widened BF16).
// normalized (optional, layer_norm only): [rows][K] BF16 of the normalised values.
void quantize_rows(const uint16_t* x, std::size_t rows, std::size_t K, Prologue prologue,
                   const uint16_t* gain, const uint16_t* bias, int8_t* q, float* scales,
                   uint16_t* normalized, uint32_t* error, hipStream_t stream,
                   Layout layout = Layout::rows);

// ---- quantised linear (src/scalar/packed_linear.cpp:8-30) ---------------------
struct DeviceLinear
{
    const int8_t* values = nullptr; // row tiles, see tile_weights
    const float* scales = nullptr;  // [K/256][N]
    const float* bias = nullptr;    // [N]
    std::size_t K = 0, N = 0;
};

// One-time host re-layout of canonical int8 weights [N][K] (input fastest) into
// row tiles: tile (t, b) holds rows 64t..64t+63 of block b as
// [segment 0..15][row 0..63][16 bytes], tiles ordered [N/64][K/256]. Requires
// K % 256 == 0 and N % 64 == 0. `tiled` holds K*N bytes.
void tile_weights(const int8_t* canonical, std::size_t K, std::size_t N, int8_t* tiled);

enum class LinearPath
{
    automatic,
    gemv,
    gemm,
    small // MFMA on row-major activations, at most 64 rows, K <= 2048
};

// y[m][n] = bf16(chain_b fma(dot_b, ws[b][n]*as[m][b]) + bias[n]); with a residual,
// y[m][n] = bf16(float(residual[m][n]) + float(that)). residual may alias y.
// Activations in Layout::tiles take the GEMM path.
void linear(const DeviceLinear& w, const int8_t* q, const float* scales, std::size_t M,
            uint16_t* y, const uint16_t* residual, LinearPath path, hipStream_t stream,
            Layout layout = Layout::rows);
std::size_t gemv_max_rows();
// Rows up to which the automatic path reads row-major activations (GEMV up to
// gemv_max_rows(), then the small-M MFMA GEMM where K <= 2048); above it the
// GEMM reads MFMA operand tiles.
std::size_t small_gemm_max_rows();
// Whether the automatic path gives M row-major rows of an N x K projection to
// the small-M MFMA GEMM (always for 8 < M <= small_gemm_max_rows() when
// K <= 2048; up to 1024 rows when the GEMM would leave most units idle).
bool small_gemm_chosen(std::size_t M, std::size_t N, std::size_t K);

// x [M][K] BF16 -> y [M][N] like quantize_rows + linear, with the BF8L buffer in
// a fixed per-device array (static_linear.hip) instead of caller or allocator
// memory; padded rows x K must not exceed static_linear_max_bytes(). Fails if
// an activation is not finite. Calls that overlap on one device race.
void linear_apply_static(const DeviceLinear& w, const uint16_t* x, std::size_t M, uint16_t* y, LinearPath path,
                         hipStream_t stream);
std::size_t static_linear_max_bytes();

// ---- row-wise elementwise kernels --------------------------------------------
void layer_norm_rows(const uint16_t* x, std::size_t rows, std::size_t width, const uint16_t* gain,
                     const uint16_t* bias, uint16_t* out, hipStream_t stream);
// out[r][i] = bf16(float(a[r][i]) + float(b[(r % b_period)][i])); out may alias a.
void add_rows(const uint16_t* a, const uint16_t* b, std::size_t rows, std::size_t width,
              std::size_t b_period, uint16_t* out, hipStream_t stream);
void softmax_rows(const uint16_t* x, std::size_t rows, std::size_t width, uint16_t* out,
                  uint32_t* error, hipStream_t stream);
void gelu_values(const uint16_t* x, std::size_t count, uint16_t* out, hipStream_t stream);

// Calibration (peak.hip): one streaming read of `bytes` (a multiple of 64 KiB),
// and an MFMA loop whose launch performs the returned number of int8 operations.
void probe_read(const void* data, std::size_t bytes, hipStream_t stream);
double probe_mfma(std::size_t workgroups, int iterations, hipStream_t stream);
void rotary_values(const uint16_t* x, const uint16_t* coefficients, std::size_t count,
                   uint16_t* out, hipStream_t stream);
} // namespace tsac_hip
