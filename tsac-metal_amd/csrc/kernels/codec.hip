// Feedback embeddings and the categorical bisection masses.
//
// Embedding sums follow src/common/cpu_transformer.tpp:205-224: the book-0
// embedding is copied, every later book is added with one BF16 rounding per add,
// in book order.
//
// Categorical masses follow src/format/categorical.cpp:44-142. For finite,
// nonnegative probabilities every probability_sum over a bisection half is a
// node of the balanced FTZ pair tree over the 1024 leaves (zero padding and the
// final add(+0, S) leave such sums unchanged), so one tree serves every level.
#include "codec.hpp"
#include "device_numeric.hpp"

namespace tsac_hip
{
namespace
{
// out[r] = (previous ? bf16(previous[r] + E[book][token[r]]) : E[book][token[r]]).
__global__ void embed_accumulate_kernel(const uint16_t* __restrict__ embeddings, int alphabet,
                                        int latent, const uint16_t* __restrict__ tokens,
                                        int token_stride, int book, int rows,
                                        const uint16_t* previous, uint16_t* out)
{
    const int chunks = latent / 8;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < rows * chunks; i += gridDim.x * blockDim.x)
    {
        const int r = i / chunks, c = i % chunks;
        const int token = tokens[std::size_t(r) * token_stride];
        const uint4 e = *reinterpret_cast<const uint4*>(
            embeddings + (std::size_t(book) * alphabet + token) * latent + c * 8);
        uint4 result = e;
        if (previous)
        {
            const uint4 p = *reinterpret_cast<const uint4*>(previous + std::size_t(r) * latent + c * 8);
            const uint32_t pw[4] = {p.x, p.y, p.z, p.w}, ew[4] = {e.x, e.y, e.z, e.w};
            uint32_t w[4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                const uint16_t lo = float_to_bf16(bf16_to_float(uint16_t(pw[k] & 0xffff)) +
                                                  bf16_to_float(uint16_t(ew[k] & 0xffff)));
                const uint16_t hi = float_to_bf16(bf16_to_float(uint16_t(pw[k] >> 16)) +
                                                  bf16_to_float(uint16_t(ew[k] >> 16)));
                w[k] = lo | (uint32_t(hi) << 16);
            }
            result = make_uint4(w[0], w[1], w[2], w[3]);
        }
        *reinterpret_cast<uint4*>(out + std::size_t(r) * latent + c * 8) = result;
    }
}

// Full feedback sum of `books` tokens per row: tokens[r][0..books).
__global__ void embed_sum_kernel(const uint16_t* __restrict__ embeddings, int alphabet, int latent,
                                 const uint16_t* __restrict__ tokens, int books, int rows,
                                 uint16_t* __restrict__ out)
{
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < rows * latent; i += gridDim.x * blockDim.x)
    {
        const int r = i / latent, k = i % latent;
        const uint16_t* t = tokens + std::size_t(r) * books;
        uint16_t sum = embeddings[std::size_t(t[0]) * latent + k];
        for (int b = 1; b < books; ++b)
        {
            const uint16_t e = embeddings[(std::size_t(b) * alphabet + t[b]) * latent + k];
            sum = float_to_bf16(bf16_to_float(sum) + bf16_to_float(e));
        }
        out[i] = sum;
    }
}

// Codebook-stack prefixes for every (step, book) row of a token block laid out
// [steps][books]: row (s, 0) is zero (it is replaced by the temporal output),
// row (s, b) is the running sum of books 0..b-1.
__global__ void embed_prefix_kernel(const uint16_t* __restrict__ embeddings, int alphabet,
                                    int latent, const uint16_t* __restrict__ tokens, int books,
                                    int steps, uint16_t* __restrict__ out)
{
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < steps * latent; i += gridDim.x * blockDim.x)
    {
        const int s = i / latent, k = i % latent;
        const uint16_t* t = tokens + std::size_t(s) * books;
        uint16_t* o = out + std::size_t(s) * books * latent + k;
        o[0] = 0;
        uint16_t sum = 0;
        for (int b = 1; b < books; ++b)
        {
            const uint16_t e = embeddings[(std::size_t(b - 1) * alphabet + t[b - 1]) * latent + k];
            sum = b == 1 ? e : float_to_bf16(bf16_to_float(sum) + bf16_to_float(e));
            o[std::size_t(b) * latent] = sum;
        }
    }
}

// dst[r] = src[r] for rows r = i * stride + offset.
__global__ void scatter_rows_kernel(const uint16_t* __restrict__ src, int rows, int width,
                                    int stride, int offset, uint16_t* __restrict__ dst)
{
    const int chunks = width / 8;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < rows * chunks; i += gridDim.x * blockDim.x)
    {
        const int r = i / chunks, c = i % chunks;
        *reinterpret_cast<uint4*>(dst + (std::size_t(r) * stride + offset) * width + c * 8) =
            *reinterpret_cast<const uint4*>(src + std::size_t(r) * width + c * 8);
    }
}

// dst[dst_index[i]] = src[src_index[i]] rows.
__global__ void copy_rows_kernel(const uint16_t* __restrict__ src, const int* __restrict__ src_index,
                                 uint16_t* __restrict__ dst, const int* __restrict__ dst_index,
                                 int rows, int width)
{
    const int chunks = width / 8;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < rows * chunks; i += gridDim.x * blockDim.x)
    {
        const int r = i / chunks, c = i % chunks;
        *reinterpret_cast<uint4*>(dst + std::size_t(dst_index[r]) * width + c * 8) =
            *reinterpret_cast<const uint4*>(src + std::size_t(src_index[r]) * width + c * 8);
    }
}

// conditional_q15 (src/format/categorical.cpp:76-89).
__device__ __forceinline__ uint16_t q15(float left, float mass)
{
    const float value = ftz_divide(ftz_multiply(left, 32768.0f), mass);
    if (!is_finite(value) || value >= 0x1p63f || value < -0x1p63f)
    {
        return 1;
    }
    const long long integer = static_cast<long long>(__builtin_rintf(value));
    const int low = int(uint32_t(uint64_t(integer)));
    return uint16_t(low < 1 ? 1 : (low > 32767 ? 32767 : low));
}

// One wavefront per 1024-entry distribution; lane l owns leaves 16l..16l+15.
// After the in-lane levels, node values for sizes 2..16 live in `local`; the
// butterfly levels give sizes 32..1024 in `wide`.
struct Tree
{
    float local[15]; // size-2 nodes [0..7], size-4 [8..11], size-8 [12..13], size-16 [14]
    float wide[6];   // sizes 32, 64, ..., 1024 (every lane of the aligned group holds it)
    bool valid;
};

__device__ __forceinline__ void build_tree(const uint16_t* row, int lane, Tree& t)
{
    const uint4 a = reinterpret_cast<const uint4*>(row + lane * 16)[0];
    const uint4 b = reinterpret_cast<const uint4*>(row + lane * 16)[1];
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float leaf[16];
    bool valid = true;
#pragma unroll
    for (int i = 0; i < 8; ++i)
    {
        leaf[2 * i] = bf16_to_float(uint16_t(w[i] & 0xffff));
        leaf[2 * i + 1] = bf16_to_float(uint16_t(w[i] >> 16));
    }
#pragma unroll
    for (int i = 0; i < 16; ++i)
    {
        valid = valid && is_finite(leaf[i]) && leaf[i] >= 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
    {
        t.local[i] = ftz_add(leaf[2 * i], leaf[2 * i + 1]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        t.local[8 + i] = ftz_add(t.local[2 * i], t.local[2 * i + 1]);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
    {
        t.local[12 + i] = ftz_add(t.local[8 + 2 * i], t.local[8 + 2 * i + 1]);
    }
    t.local[14] = ftz_add(t.local[12], t.local[13]);
    float v = t.local[14];
    t.wide[0] = v = butterfly_ftz_add<1>(v);
    t.wide[1] = v = butterfly_ftz_add<2>(v);
    t.wide[2] = v = butterfly_ftz_add<4>(v);
    t.wide[3] = v = butterfly_ftz_add<8>(v);
    t.wide[4] = v = butterfly_ftz_add<16>(v);
    t.wide[5] = v = butterfly_ftz_add<32>(v);
    t.valid = __all(valid);
    (void)leaf;
}

// Mass of the aligned node [base, base + size) (size a power of two <= 512).
__device__ __forceinline__ float node_mass(const Tree& t, int base, int size, const uint16_t* row)
{
    const int owner = base / 16;
    float mine;
    if (size >= 32)
    {
        int level = 0;
        for (int s = 32; s < size; s *= 2)
        {
            ++level;
        }
        mine = t.wide[0];
#pragma unroll
        for (int l = 1; l < 6; ++l)
        {
            mine = l == level ? t.wide[l] : mine;
        }
    }
    else
    {
        const int offset = base % 16;
        int index;
        if (size == 16)
        {
            index = 14;
        }
        else if (size == 8)
        {
            index = 12 + offset / 8;
        }
        else if (size == 4)
        {
            index = 8 + offset / 4;
        }
        else if (size == 2)
        {
            index = offset / 2;
        }
        else
        {
            index = -1;
        }
        mine = 0.0f;
#pragma unroll
        for (int i = 0; i < 15; ++i)
        {
            mine = i == index ? t.local[i] : mine;
        }
        if (size == 1)
        {
            // A single leaf: pair tree over eight zero-padded slots == the leaf (flushed).
            mine = flush(bf16_to_float(row[base]));
        }
    }
    return __shfl(mine, owner, wave);
}

// Encoder side: the ten Q15 split probabilities along `symbol`'s path.
__global__ __launch_bounds__(256) void categorical_path_kernel(const uint16_t* __restrict__ probs,
                                                               int rows, int alphabet,
                                                               const uint16_t* __restrict__ symbols,
                                                               uint16_t* __restrict__ splits,
                                                               uint32_t* __restrict__ error)
{
    const int lane = threadIdx.x % wave;
    const int row = blockIdx.x * 4 + threadIdx.x / wave;
    if (row >= rows)
    {
        return;
    }
    const uint16_t* p = probs + std::size_t(row) * alphabet;
    Tree t;
    build_tree(p, lane, t);
    if (!t.valid)
    {
        error[0] = error_nonfinite;
    }
    const int symbol = symbols[row];
    int base = 0, count = alphabet, level = 0;
    float mass = 1.0f;
    uint16_t mine = 0;
    while (count > 1)
    {
        const int half = count / 2;
        const float left = node_mass(t, base, half, p);
        const uint16_t split = q15(left, mass);
        if (lane == level)
        {
            mine = split;
        }
        if (symbol >= base + half)
        {
            base += half;
            count -= half;
            mass = flush(flush(mass) - flush(left));
        }
        else
        {
            count = half;
            mass = left;
        }
        ++level;
    }
    if (lane < level)
    {
        splits[std::size_t(row) * 16 + lane] = mine;
    }
}

// Decoder side: all internal node masses in heap order (node 1 = root,
// children 2i and 2i+1); entry 0 carries the validity flag (1.0f = valid).
__global__ __launch_bounds__(256) void categorical_tree_kernel(const uint16_t* __restrict__ probs,
                                                               int rows, float* __restrict__ nodes)
{
    const int lane = threadIdx.x % wave;
    const int row = blockIdx.x * 4 + threadIdx.x / wave;
    if (row >= rows)
    {
        return;
    }
    Tree t;
    build_tree(probs + std::size_t(row) * 1024, lane, t);
    float* n = nodes + std::size_t(row) * 1024;
    // Leaves of lane l are 16l..16l+15; heap index of a size-s node starting at
    // leaf x is (1024 / s) + x / s.
#pragma unroll
    for (int i = 0; i < 8; ++i)
    {
        n[512 + (lane * 16 + 2 * i) / 2] = t.local[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        n[256 + (lane * 16 + 4 * i) / 4] = t.local[8 + i];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
    {
        n[128 + (lane * 16 + 8 * i) / 8] = t.local[12 + i];
    }
    n[64 + lane] = t.local[14];
#pragma unroll
    for (int level = 0; level < 6; ++level)
    {
        const int size = 32 << level;
        if ((lane * 16) % size == 0)
        {
            n[1024 / size + lane * 16 / size] = t.wide[level];
        }
    }
    if (lane == 0)
    {
        n[0] = t.valid ? 1.0f : 0.0f;
    }
}

unsigned grid_for(std::size_t items)
{
    const std::size_t blocks = (items + 255) / 256;
    return unsigned(blocks == 0 ? 1 : (blocks < 16384 ? blocks : 16384));
}
} // namespace

void embed_accumulate(const uint16_t* embeddings, std::size_t alphabet, std::size_t latent,
                      const uint16_t* tokens, std::size_t token_stride, std::size_t book,
                      std::size_t rows, const uint16_t* previous, uint16_t* out, hipStream_t stream)
{
    require(latent % 8 == 0, "embedding width must be a multiple of 8");
    if (!rows)
    {
        return;
    }
    embed_accumulate_kernel<<<grid_for(rows * latent / 8), 256, 0, stream>>>(
        embeddings, int(alphabet), int(latent), tokens, int(token_stride), int(book), int(rows),
        previous, out);
    check_hip(hipGetLastError(), "embed launch");
}

void embed_sum(const uint16_t* embeddings, std::size_t alphabet, std::size_t latent,
               const uint16_t* tokens, std::size_t books, std::size_t rows, uint16_t* out,
               hipStream_t stream)
{
    require(books >= 1, "embedding needs at least one book");
    if (!rows)
    {
        return;
    }
    embed_sum_kernel<<<grid_for(rows * latent), 256, 0, stream>>>(embeddings, int(alphabet), int(latent),
                                                                  tokens, int(books), int(rows), out);
    check_hip(hipGetLastError(), "embed launch");
}

void embed_prefixes(const uint16_t* embeddings, std::size_t alphabet, std::size_t latent,
                    const uint16_t* tokens, std::size_t books, std::size_t steps, uint16_t* out,
                    hipStream_t stream)
{
    if (!steps)
    {
        return;
    }
    embed_prefix_kernel<<<grid_for(steps * latent), 256, 0, stream>>>(
        embeddings, int(alphabet), int(latent), tokens, int(books), int(steps), out);
    check_hip(hipGetLastError(), "embed prefix launch");
}

void scatter_rows(const uint16_t* src, std::size_t rows, std::size_t width, std::size_t stride,
                  std::size_t offset, uint16_t* dst, hipStream_t stream)
{
    require(width % 8 == 0, "row width must be a multiple of 8");
    if (!rows)
    {
        return;
    }
    scatter_rows_kernel<<<grid_for(rows * width / 8), 256, 0, stream>>>(src, int(rows), int(width),
                                                                        int(stride), int(offset), dst);
    check_hip(hipGetLastError(), "scatter launch");
}

void copy_rows(const uint16_t* src, const int* src_index, uint16_t* dst, const int* dst_index,
               std::size_t rows, std::size_t width, hipStream_t stream)
{
    require(width % 8 == 0, "row width must be a multiple of 8");
    if (!rows)
    {
        return;
    }
    copy_rows_kernel<<<grid_for(rows * width / 8), 256, 0, stream>>>(src, src_index, dst, dst_index,
                                                                     int(rows), int(width));
    check_hip(hipGetLastError(), "copy rows launch");
}

void categorical_paths(const uint16_t* probs, std::size_t rows, std::size_t alphabet,
                       const uint16_t* symbols, uint16_t* splits, uint32_t* error, hipStream_t stream)
{
    require(alphabet == 1024, "categorical kernels need a 1024-symbol alphabet");
    if (!rows)
    {
        return;
    }
    categorical_path_kernel<<<unsigned((rows + 3) / 4), 256, 0, stream>>>(probs, int(rows), int(alphabet),
                                                                         symbols, splits, error);
    check_hip(hipGetLastError(), "categorical path launch");
}

void categorical_trees(const uint16_t* probs, std::size_t rows, float* nodes, hipStream_t stream)
{
    if (!rows)
    {
        return;
    }
    categorical_tree_kernel<<<unsigned((rows + 3) / 4), 256, 0, stream>>>(probs, int(rows), nodes);
    check_hip(hipGetLastError(), "categorical tree launch");
}
} // namespace tsac_hip
