// Frame-step kernel (frame.hpp). Every job computes exactly what the matching
// decode kernel in decode.hip computes, in the same order (BF8L quantiser,
// LayerNorm, exact int8 block dots and ordered per-block fma chain of
// src/scalar/packed_linear.cpp:16-27, attention recurrence of
// src/scalar/attention.cpp:62-101, softmax of src/common/probability.cpp:96-122,
// categorical bisection of src/format/categorical.cpp:119-142 with the range
// decoder of src/format/range.cpp:131-151); only where its inputs come from and
// where its outputs go differ.
#include "frame.hpp"
#include "row_ops.hpp"
#include "step_ops.hpp"

#include <algorithm>
#include <array>
#include <atomic>
#include <cstring>

namespace tsac_hip
{
namespace
{
using namespace step;
using word = unsigned long long;

constexpr int frame_waves = 8;
constexpr int frame_threads = frame_waves * wave;
// Waves that take, normalise and quantise a projection's spread input row
// (K = 64 V values): fewer waves mean fewer barriers and no two of them
// sharing a SIMD, against more values per lane. Measured per frame step of the
// 2580-frame decode: 2 waves for K <= 512 (no BF8L exchange, one LayerNorm
// exchange) 704 us, 1 wave 718 us, 8 waves 731 us; 8 waves for K = 2048, 4
// waves 721 us. K = 1024 (the 1024-wide geometry): 4 waves of 4 values, one
// BF8L block per wave, 1,195.6 us; 8 waves 1,210.5 us; 2 waves 1,228.4 us.
template <int V> constexpr int spread_waves = V <= 8 ? 2 : V <= 16 ? 4 : 8;
constexpr int max_lanes = 8;
// Output rows of a narrow projection tile (project_tile, FrameLayout::narrow_down).
constexpr int narrow_rows = tile_rows / 2;
constexpr int max_blocks = 16; // 64-key blocks of one attention query (context <= 1024)
constexpr int max_books = 16;  // codebook positions of one frame
// Polls of one word before a wait is declared stalled (each poll sleeps ~64
// clocks and makes one device-scope load): seconds, far beyond any real wait.
constexpr unsigned spin_limit = 1u << 22;

// Jobs pass nothing between their waves through global memory, so their
// barriers are lds_barrier() (row_ops.hpp): the next job's weight prefetch and
// the words just published are not waited for.

// ------------------------------------------------------------------ exchange words

struct Exchange
{
    uint32_t epoch;
    unsigned* abort;
};

// Global-address views: job arguments reach the jobs through memory, so their
// pointers are generic; these keep the accesses global, not flat. A flat access
// counts against both the vector-memory and the LDS counters, so every later
// wait for the wave's LDS accesses would also wait for it (for a store, until
// memory acknowledges it).
template <class T> __device__ __forceinline__ const __attribute__((address_space(1))) T* global(const T* p)
{
    return (const __attribute__((address_space(1))) T*)(p);
}
template <class T> __device__ __forceinline__ __attribute__((address_space(1))) T* global_out(T* p)
{
    return (__attribute__((address_space(1))) T*)(p);
}

__device__ __forceinline__ void publish(word* w, std::size_t index, uint32_t payload, uint32_t epoch)
{
    __hip_atomic_store(global_out(w + index), (word(epoch) << 32) | payload, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// V consecutive BF16 values of a row in global memory (p aligned to V values).
template <int V> __device__ __forceinline__ void load_global_row(const uint16_t* p, uint16_t (&v)[V])
{
    if constexpr (V == 1)
    {
        v[0] = *global(p);
    }
    else if constexpr (V == 2)
    {
        const uint32_t u = *global(reinterpret_cast<const uint32_t*>(p));
        v[0] = uint16_t(u & 0xffff), v[1] = uint16_t(u >> 16);
    }
    else
    {
        static_assert(V % 4 == 0, "1, 2 or a multiple of 4 values");
#pragma unroll
        for (int c = 0; c < V / 4; ++c)
        {
            const unsigned long long u = *global(reinterpret_cast<const unsigned long long*>(p) + c);
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                v[4 * c + i] = uint16_t(u >> (16 * i));
            }
        }
    }
}

// The workgroup's LDS block as a pointer the compiler knows to be in LDS (job
// functions receive it as a generic pointer), so that the accesses through it
// are LDS instructions rather than flat ones.
__device__ __forceinline__ uint8_t* in_lds(uint8_t* p)
{
    return (uint8_t*)((__attribute__((address_space(3))) uint8_t*)(p));
}

// Job functions stay out of line (each is one body in the instruction cache)
// and are never tail-called: LLVM then gives these internal, non-recursive
// functions no callee-saved registers (the kernel saves what it keeps live),
// instead of saving and restoring up to ~100 registers in private memory on
// every job.
#define JOB __attribute__((not_tail_called))

// Job descriptors live in a device table written before the launch and never
// during it (frame_job_table), read through the constant address space so
// every field is a scalar load into scalar registers.
template <class T> using constant_ptr = const __attribute__((address_space(4))) T*;
template <class T> __device__ __forceinline__ constant_ptr<T> constant(const void* p)
{
    return (constant_ptr<T>)(p);
}

// Job arguments reach each job through memory, so the compiler cannot see that
// they are the same in every lane; these move them into scalar registers (and
// make branches on them scalar).
__device__ __forceinline__ int uniform(int v)
{
    return __builtin_amdgcn_readfirstlane(v);
}
__device__ __forceinline__ std::size_t uniform(std::size_t v)
{
    const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(v)), hi = __builtin_amdgcn_readfirstlane(uint32_t(v >> 32));
    return (std::size_t(hi) << 32) | lo;
}
__device__ __forceinline__ long long uniform(long long v)
{
    return static_cast<long long>(uniform(static_cast<std::size_t>(v)));
}
__device__ __forceinline__ float uniform(float v)
{
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
template <class T> __device__ __forceinline__ T* uniform(T* p)
{
    return reinterpret_cast<T*>(uniform(reinterpret_cast<std::size_t>(p)));
}

// Keeps a value in vector registers: a value every lane loads from one shared
// address is otherwise kept in scalar registers, and the compiler then spills
// such values into vector-register lanes and reads each back with readlane
// and a wait.
__device__ __forceinline__ void in_vgprs(float4& u)
{
    asm volatile("" : "+v"(u.x), "+v"(u.y), "+v"(u.z), "+v"(u.w));
}

// Row stride (floats) of the codebook keys staged in fp32: 16 bytes of padding
// move consecutive rows four banks apart, so lane r reading row r at the same
// column hits distinct banks.
template <int HW> constexpr int staged_key_stride = HW + 4;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint4 load16(const void* p)
{
    const u32x4 v = *global(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float2 load_float2(const float* p)
{
    const f32x2 v = *global(reinterpret_cast<const f32x2*>(p));
    return make_float2(v.x, v.y);
}

__device__ __forceinline__ word peek(const word* w, std::size_t index)
{
    return __hip_atomic_load(global(w + index), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// This lane's V consecutive BF16 values of a row in (global) memory.
template <int V> __device__ __forceinline__ void load_values(const uint16_t* p, uint16_t (&v)[V])
{
    static_assert(V % 8 == 0, "whole 16-byte chunks");
#pragma unroll
    for (int c = 0; c < V / 8; ++c)
    {
        const uint4 u = load16(p + 8 * c);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            v[8 * c + 2 * i] = uint16_t(w[i] & 0xffff);
            v[8 * c + 2 * i + 1] = uint16_t(w[i] >> 16);
        }
    }
}

// Payload of word `index` once it carries the epoch; `seen` is a value already
// loaded. After a stall (or once any wait has stalled) returns 0 at once.
__device__ __forceinline__ bool keep_polling(unsigned& spins, const Exchange& x);
__device__ __forceinline__ uint32_t settle(const word* w, std::size_t index, word seen, const Exchange& x)
{
    unsigned spins = 0;
    while (uint32_t(seen >> 32) != x.epoch)
    {
        if (!keep_polling(spins, x))
        {
            return 0u;
        }
        seen = peek(w, index);
    }
    return uint32_t(seen);
}

__device__ __forceinline__ uint32_t take(const word* w, std::size_t index, const Exchange& x)
{
    return settle(w, index, peek(w, index), x);
}

// Gives up on a wait after too many polls (raising the abort word) or once
// another wait has; true while polling should go on.
__device__ __forceinline__ bool keep_polling(unsigned& spins, const Exchange& x)
{
    if (++spins % 64 == 0)
    {
        if (__hip_atomic_load(global_out(x.abort), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u)
        {
            return false;
        }
        if (spins > spin_limit)
        {
            __hip_atomic_store(global_out(x.abort), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
    }
    // Short waits poll at once; long ones back off, which keeps the many
    // workgroups waiting for later jobs from crowding memory.
    if (spins < 32)
    {
        __builtin_amdgcn_s_sleep(1);
    }
    else if (spins < 128)
    {
        __builtin_amdgcn_s_sleep(4);
    }
    else
    {
        __builtin_amdgcn_s_sleep(12);
    }
    return true;
}

// Payloads of N words, at address(i) for word i, once each carries the epoch.
// Each poll requests all N words before it waits for any (a load under a
// per-word branch would wait for its own reply, making a poll N round trips);
// words already current keep their first value.
template <int N, class Address>
__device__ __forceinline__ void take_words(const Address& address, const Exchange& x, uint32_t (&out)[N])
{
    static_assert(N <= 64, "one pending mask");
    unsigned long long pending = N == 64 ? ~0ull : (1ull << N) - 1;
    unsigned spins = 0;
    do
    {
        word v[N];
#pragma unroll
        for (int i = 0; i < N; ++i)
        {
            v[i] = __hip_atomic_load(global(address(i)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int i = 0; i < N; ++i)
        {
            if (((pending >> i) & 1ull) && uint32_t(v[i] >> 32) == x.epoch)
            {
                out[i] = uint32_t(v[i]);
                pending &= ~(1ull << i);
            }
        }
    } while (pending && keep_polling(spins, x));
}

// Device-coherent 16-byte loads of Q consecutive chunks at p (16-byte
// aligned), all requested before the one wait for their replies. One asm
// statement, so no instruction can read a destination before the data is in:
// left to itself the compiler may issue such loads one at a time, each with
// its own wait, which makes a poll of a long row many round trips. sc1 is the
// cache policy of the compiler's own agent-scope atomic loads; each 8-byte
// word of a chunk is read whole, as its producer wrote it.
#define TSAC_CHUNK(n, offset) "global_load_dwordx4 %" #n ", %[at], off offset:" #offset " sc1\n"
template <int Q> __device__ __forceinline__ void load_chunks(const word* p, u32x4 (&c)[Q])
{
    if constexpr (Q == 2)
    {
        asm volatile(TSAC_CHUNK(0, 0) TSAC_CHUNK(1, 16) "s_waitcnt vmcnt(0)"
                     : "=&v"(c[0]), "=&v"(c[1])
                     : [at] "v"(p)
                     : "memory");
    }
    else if constexpr (Q == 4)
    {
        asm volatile(TSAC_CHUNK(0, 0) TSAC_CHUNK(1, 16) TSAC_CHUNK(2, 32) TSAC_CHUNK(3, 48) "s_waitcnt vmcnt(0)"
                     : "=&v"(c[0]), "=&v"(c[1]), "=&v"(c[2]), "=&v"(c[3])
                     : [at] "v"(p)
                     : "memory");
    }
    else if constexpr (Q == 8)
    {
        asm volatile(TSAC_CHUNK(0, 0) TSAC_CHUNK(1, 16) TSAC_CHUNK(2, 32) TSAC_CHUNK(3, 48) TSAC_CHUNK(4, 64)
                         TSAC_CHUNK(5, 80) TSAC_CHUNK(6, 96) TSAC_CHUNK(7, 112) "s_waitcnt vmcnt(0)"
                     : "=&v"(c[0]), "=&v"(c[1]), "=&v"(c[2]), "=&v"(c[3]), "=&v"(c[4]), "=&v"(c[5]), "=&v"(c[6]),
                       "=&v"(c[7])
                     : [at] "v"(p)
                     : "memory");
    }
    else
    {
        static_assert(Q == 16, "2, 4, 8 or 16 chunks");
        asm volatile(TSAC_CHUNK(0, 0) TSAC_CHUNK(1, 16) TSAC_CHUNK(2, 32) TSAC_CHUNK(3, 48) TSAC_CHUNK(4, 64)
                         TSAC_CHUNK(5, 80) TSAC_CHUNK(6, 96) TSAC_CHUNK(7, 112) TSAC_CHUNK(8, 128)
                             TSAC_CHUNK(9, 144) TSAC_CHUNK(10, 160) TSAC_CHUNK(11, 176) TSAC_CHUNK(12, 192)
                                 TSAC_CHUNK(13, 208) TSAC_CHUNK(14, 224) TSAC_CHUNK(15, 240) "s_waitcnt vmcnt(0)"
                     : "=&v"(c[0]), "=&v"(c[1]), "=&v"(c[2]), "=&v"(c[3]), "=&v"(c[4]), "=&v"(c[5]), "=&v"(c[6]),
                       "=&v"(c[7]), "=&v"(c[8]), "=&v"(c[9]), "=&v"(c[10]), "=&v"(c[11]), "=&v"(c[12]),
                       "=&v"(c[13]), "=&v"(c[14]), "=&v"(c[15])
                     : [at] "v"(p)
                     : "memory");
    }
}
#undef TSAC_CHUNK

// This lane's V consecutive BF16 values starting at value `first` of a word
// vector (first a multiple of 4, the vector 16-byte aligned), once every word
// carries the epoch. Words already current keep their first value.
template <int V>
__device__ __forceinline__ void take_row(const word* w, std::size_t first, const Exchange& x, uint16_t (&v)[V])
{
    static_assert(V % 4 == 0, "whole 16-byte chunks");
    constexpr int words = V / 2, chunks = V / 4;
    const word* p = w + first / 2;
    uint32_t got[words];
    unsigned long long pending = words == 64 ? ~0ull : (1ull << words) - 1;
    unsigned spins = 0;
    do
    {
        u32x4 c[chunks];
        load_chunks<chunks>(p, c);
#pragma unroll
        for (int j = 0; j < chunks; ++j)
        {
            const uint32_t payload[2] = {c[j].x, c[j].z}, epoch[2] = {c[j].y, c[j].w};
#pragma unroll
            for (int h = 0; h < 2; ++h)
            {
                const int i = 2 * j + h;
                if (((pending >> i) & 1ull) && epoch[h] == x.epoch)
                {
                    got[i] = payload[h];
                    pending &= ~(1ull << i);
                }
            }
        }
    } while (pending && keep_polling(spins, x));
#pragma unroll
    for (int i = 0; i < words; ++i)
    {
        v[2 * i] = uint16_t(got[i] & 0xffff);
        v[2 * i + 1] = uint16_t(got[i] >> 16);
    }
}

// This lane's Vw consecutive BF16 values from value `first` (a multiple of Vw)
// of a word vector, once current; with Vw == 1 neighbouring lanes share a word.
template <int Vw>
__device__ __forceinline__ void take_values(const word* w, std::size_t first, const Exchange& x, uint16_t (&v)[Vw])
{
    constexpr int words = Vw < 2 ? 1 : Vw / 2;
    uint32_t got[words];
    take_words<words>([&](int i) -> const word* { return w + first / 2 + i; }, x, got);
    if constexpr (Vw == 1)
    {
        v[0] = uint16_t((first & 1) ? got[0] >> 16 : got[0] & 0xffffu);
    }
    else
    {
#pragma unroll
        for (int i = 0; i < words; ++i)
        {
            v[2 * i] = uint16_t(got[i] & 0xffffu);
            v[2 * i + 1] = uint16_t(got[i] >> 16);
        }
    }
}

template <int V>
__device__ __forceinline__ void give_row(word* w, std::size_t first, const Exchange& x, const uint16_t (&v)[V])
{
#pragma unroll
    for (int i = 0; i < V / 2; ++i)
    {
        publish(w, first / 2 + i, v[2 * i] | (uint32_t(v[2 * i + 1]) << 16), x.epoch);
    }
}

// ------------------------------------------------------------------ exchange layout

// Word offsets of every exchanged matrix of one step, rows of 8 lanes, row m of
// an N-wide matrix at m*N/2.
struct Words
{
    std::size_t w, qkv, hid, logit, pre, layer, temporal, book, records, record_layer, total;

    __host__ __device__ Words(int width, int ffn, int latent, int alphabet, int books, int temporal_layers,
                               int codebook_layers)
    {
        w = 4 * std::size_t(width);
        qkv = 12 * std::size_t(width);
        hid = 4 * std::size_t(ffn);
        logit = 4 * std::size_t(alphabet);
        pre = 4 * std::size_t(latent);
        layer = qkv + w + w + hid + w; // qkv, attention, mid residual, hidden, out
        temporal = w + temporal_layers * layer;
        book = pre + w + codebook_layers * layer + logit + 8;
        // Block records of the temporal attention's second half (blocks 8-15)
        // per layer: max_lanes lanes x heads x 8 blocks x (2 + head width)
        // words, with heads <= width / 64.
        records = temporal + std::size_t(books) * book;
        record_layer = std::size_t(max_lanes) * 8 * (std::size_t(width) + width / 32);
        total = records + std::size_t(temporal_layers) * record_layer;
    }
    __host__ __device__ std::size_t t_records(int l) const
    {
        return records + l * record_layer;
    }
    // Temporal stack: input of layer l (l == layers is its output).
    __host__ __device__ std::size_t t_x(int l) const
    {
        return l == 0 ? 0 : w + (l - 1) * layer + qkv + w + w + hid;
    }
    __host__ __device__ std::size_t t_qkv(int l) const
    {
        return w + l * layer;
    }
    __host__ __device__ std::size_t t_att(int l) const
    {
        return t_qkv(l) + qkv;
    }
    __host__ __device__ std::size_t t_mid(int l) const
    {
        return t_att(l) + w;
    }
    __host__ __device__ std::size_t t_hid(int l) const
    {
        return t_mid(l) + w;
    }
    __host__ __device__ std::size_t c_base(int b) const
    {
        return temporal + b * book;
    }
    __host__ __device__ std::size_t c_prefix(int b) const
    {
        return c_base(b);
    }
    __host__ __device__ std::size_t c_x(int b, int l) const
    {
        return l == 0 ? c_base(b) + pre : c_base(b) + pre + w + (l - 1) * layer + qkv + w + w + hid;
    }
    __host__ __device__ std::size_t c_qkv(int b, int l) const
    {
        return c_base(b) + pre + w + l * layer;
    }
    __host__ __device__ std::size_t c_att(int b, int l) const
    {
        return c_qkv(b, l) + qkv;
    }
    __host__ __device__ std::size_t c_mid(int b, int l) const
    {
        return c_att(b, l) + w;
    }
    __host__ __device__ std::size_t c_hid(int b, int l) const
    {
        return c_mid(b, l) + w;
    }
    __host__ __device__ std::size_t c_logits(int b, int codebook_layers) const
    {
        return c_base(b) + pre + w + codebook_layers * layer;
    }
    __host__ __device__ std::size_t c_token(int b, int codebook_layers) const
    {
        return c_logits(b, codebook_layers) + logit;
    }
};

// ------------------------------------------------------------------ projection job

enum class In
{
    words,            // BF16 rows from exchange words
    words_norm,       // LayerNorm of those rows
    embed_sum,        // sum of the previous frame's feedback embeddings (memory tokens)
    embed_accumulate, // prefix (words) + embedding of the previous book's token (words)
    attention,        // codebook attention of the lane over its books (from the qkv words)
};

enum class Out
{
    plain,          // y
    residual_words, // bf16(residual row from words + y)
    residual_row,   // bf16(one memory row + y)
    gelu,           // gelu(y)
    qkv,            // rotary on Q and K, all three exchanged, K and V also into the cache
};

struct Projection
{
    DeviceLinear w;
    const word* x = nullptr;
    const uint16_t* gain = nullptr;
    const uint16_t* beta = nullptr;
    const uint16_t* embeddings = nullptr;
    int alphabet = 0, books = 0, book = 0;
    const uint16_t* tokens = nullptr; // embed_sum: [lanes][token_stride]
    int token_stride = 0;
    // embed_accumulate: previous book's tokens; embed_sum: book 0's tokens,
    // book b's at + b * token_book_words (the previous step's, within a launch)
    const word* token_words = nullptr;
    std::size_t token_book_words = 0;
    const word* prefix_in = nullptr;   // embed_accumulate: previous prefix (null for the first)
    word* prefix_out = nullptr;        // embed_accumulate: published by tile 0
    const word* residual = nullptr;
    const uint16_t* residual_row = nullptr;
    word* y = nullptr;
    int position = 0;
    const uint16_t* rotations = nullptr;
    int width = 0, head_width = 0;
};

// In::attention: the layer's qkv words of book 0 (book t at + t*book_words),
// keys 0 .. time-1, and the one lane whose row the tile computes.
struct BookAttention
{
    const word* qkv = nullptr;
    std::size_t book_words = 0;
    int time = 0, lane = 0;
    float scale = 0.0f;
};

// A projection's LDS: quantised rows, their block scales, the partial dots,
// then the exchange words of the spread LayerNorm (2 per wave) and BF8L (1 per
// wave).
template <int V> constexpr int projection_exchange()
{
    constexpr int K = wave * V, blocks = K / 256, slots = blocks > frame_waves ? blocks : frame_waves;
    return max_lanes * K + max_lanes * blocks * 4 + slots * max_lanes * tile_rows * 4;
}
template <int V> constexpr int projection_lds()
{
    return projection_exchange<V>() + 3 * frame_waves * 4;
}

// ------------------------------------------------------------------ codebook attention in a projection

// LDS (floats) of one wave's codebook attention head: the fp32 query, the
// fp32 keys (padded rows), the value words and the query's weights.
template <int HW> constexpr int book_head_floats = HW + max_books * staged_key_stride<HW> + max_books * HW / 2 + wave;

// A projection computes codebook attention rows when each wave has at most
// two heads (width / HW <= 2 * frame_waves; wave w takes heads w and
// w + frame_waves): per-head regions, then the lane's BF16 attention row,
// after the projection's own LDS.
constexpr int max_book_heads_per_wave = 2;
template <int V, int HW> constexpr int book_heads = HW > 0 ? wave * V / HW : 0;
template <int V, int HW>
constexpr bool book_attention_fits = HW > 0 && book_heads<V, HW> <= max_book_heads_per_wave * frame_waves;
template <int V, int HW> constexpr int book_attention_lds()
{
    return book_attention_fits<V, HW> ? book_heads<V, HW> * book_head_floats<HW> * 4 + wave * V * 2 : 0;
}

// The `count` (<= H) codebook attention heads head0, head0 + frame_waves, ...
// of lane m over keys 0 .. time-1 (time <= max_books: one block of
// attend_item, which computes the same values in the same order) by one wave;
// head h is staged in regions + h * book_head_floats<HW> and its BF16 outputs
// go to row[h*HW ...]. The books before the current one were published long
// before this job, so the key and value words of all the wave's heads for
// those books are requested first, and only then are the current book's
// query, key and value words polled for.
// A thread given `residual` also requests that word as soon as the current
// book's words are in (the residual row is the layer's input, which the qkv
// job consumed before it published them), into `residual_seen`.
template <int HW, int H>
__device__ __forceinline__ void wave_book_heads(const word* qkv, std::size_t book_words, int time, int width,
                                                float scale, int m, int head0, int count, const Exchange& x,
                                                float* regions, uint16_t* row, const word* residual,
                                                word& residual_seen)
{
    constexpr int per_lane = HW / 64, key_stride = staged_key_stride<HW>;
    const int lane = threadIdx.x % wave;
    // Staging of head h: the fp32 query [HW], fp32 keys [max_books][key_stride],
    // value words [max_books][HW/2], the query's weights [wave].
    const auto query_of = [&](int h) { return regions + h * book_head_floats<HW>; };
    const auto keys_of = [&](int h) { return query_of(h) + HW; };
    const auto values_of = [&](int h) { return reinterpret_cast<uint32_t*>(keys_of(h) + max_books * key_stride); };
    const auto head_of = [&](int k) { return head0 + k * frame_waves; };
    // Word of value index head*HW of lane m's qkv row: query, then key (+width/2), value (+width).
    const auto query_word = [&](int h) { return (std::size_t(m) * 3 * width + std::size_t(h) * HW) / 2; };
    const auto pair = [](uint32_t w) { return make_float2(__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u)); };

    // 1. Earlier books, four at a time for all the wave's heads (one request
    //    of all their words each): word i of (book r, head) is key word i for
    //    i < HW/2, else value word i - HW/2.
    const int older = (time - 1) * HW; // words per head
    constexpr int chunk = 4 * HW, per_thread = H * chunk / wave;
    for (int first = 0; first < older; first += chunk)
    {
        uint32_t got[per_thread];
        // Word i of this lane: head k, offset o of that head's earlier words.
        const auto locate = [&](int i, int& k, int& o)
        {
            const int w = lane + i * wave;
            k = w / chunk;
            o = first + w % chunk;
            return k < count && o < older;
        };
        const auto address = [&](int i) -> const word*
        {
            int k, o;
            if (!locate(i, k, o))
            {
                k = 0;
                o = first;
            }
            const int r = o / HW, c = o % HW;
            const std::size_t q = query_word(head_of(k));
            return qkv + std::size_t(r) * book_words + (c < HW / 2 ? q + width / 2 + c : q + width + (c - HW / 2));
        };
        take_words<per_thread>(address, x, got);
#pragma unroll
        for (int i = 0; i < per_thread; ++i)
        {
            int k, o;
            if (locate(i, k, o))
            {
                const int h = head_of(k), r = o / HW, c = o % HW;
                if (c < HW / 2)
                {
                    reinterpret_cast<float2*>(keys_of(h) + r * key_stride)[c] = pair(got[i]);
                }
                else
                {
                    values_of(h)[r * (HW / 2) + c - HW / 2] = got[i];
                }
            }
        }
    }
    // 2. The current book, head by head: query words, then key words, then
    //    value words.
    {
        constexpr int row_words = 3 * HW / 2, per_thread = (H * row_words + wave - 1) / wave;
        const int r = time - 1, total = count * row_words;
        const word* base = qkv + std::size_t(r) * book_words;
        uint32_t got[per_thread];
        const auto address = [&](int i) -> const word*
        {
            int w = lane + i * wave;
            w = w < total ? w : total - 1;
            const int k = w / row_words, c = w % row_words;
            const std::size_t q = query_word(head_of(k));
            return base + (c < HW / 2 ? q + c : c < HW ? q + width / 2 + (c - HW / 2) : q + width + (c - HW));
        };
        take_words<per_thread>(address, x, got);
        if (residual)
        {
            residual_seen = peek(residual, 0);
        }
#pragma unroll
        for (int i = 0; i < per_thread; ++i)
        {
            const int w = lane + i * wave;
            if (w < total)
            {
                const int h = head_of(w / row_words), c = w % row_words;
                if (c < HW / 2)
                {
                    reinterpret_cast<float2*>(query_of(h))[c] = pair(got[i]);
                }
                else if (c < HW)
                {
                    reinterpret_cast<float2*>(keys_of(h) + r * key_stride)[c - HW / 2] = pair(got[i]);
                }
                else
                {
                    values_of(h)[r * (HW / 2) + c - HW] = got[i];
                }
            }
        }
    }
    // The staged rows are read by other lanes of this wave only.
    asm volatile("" ::: "memory");
    wait_shared_memory();
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");

    if constexpr (H == 2 && HW == 64)
    {
        if (count == 2)
        {
            // Both heads at once, head head_of(h) in lanes [32h, 32h + 32): key
            // t (< time <= max_books <= 32) in lane 32h + t for the scores, and
            // value columns 2j, 2j + 1 in lane 32h + j for the sums. Each score,
            // sum and column takes the same operations in the same order as in
            // one block of attend_item; the 32-lane max and pair tree equal the
            // 64-lane ones whose upper leaves are -inf and +0.
            const int half = lane / 32, j = lane % 32, head = head_of(half);
            const float* query = query_of(head);
            const uint32_t* values = values_of(head);
            float* weights = reinterpret_cast<float*>(values_of(head) + max_books * HW / 2);
            float score = -__builtin_inff();
            if (j < time)
            {
                const float4* q4 = reinterpret_cast<const float4*>(query);
                const float4* k4 = reinterpret_cast<const float4*>(keys_of(head) + j * key_stride);
                constexpr int chunks = HW / 4, ahead = 4;
                float4 qs[ahead], ks[ahead];
#pragma unroll
                for (int c = 0; c < ahead; ++c)
                {
                    qs[c] = q4[c];
                    ks[c] = k4[c];
                }
                float dot = 0.0f;
#pragma unroll
                for (int c = 0; c < chunks; ++c)
                {
                    float4 qc = qs[c % ahead];
                    const float4 kc = ks[c % ahead];
                    if (c + ahead < chunks)
                    {
                        qs[c % ahead] = q4[c + ahead];
                        ks[c % ahead] = k4[c + ahead];
                    }
                    in_vgprs(qc);
                    dot = __builtin_fmaf(qc.x, kc.x, dot);
                    dot = __builtin_fmaf(qc.y, kc.y, dot);
                    dot = __builtin_fmaf(qc.z, kc.z, dot);
                    dot = __builtin_fmaf(qc.w, kc.w, dot);
                }
                score = dot * scale;
            }
            const float maximum = group_max<32>(score);
            float e = 0.0f;
            if (j < time)
            {
                e = original_exp(score - maximum);
            }
            const float sum = tree_sum<32>(e);
            weights[j] = e;
            asm volatile("" ::: "memory");
            wait_shared_memory();
            __builtin_amdgcn_wave_barrier();
            asm volatile("" ::: "memory");
            // Every key's weight and value word is requested before the first
            // is used (rows past `time` hold stale words, and their steps are
            // dropped by selects, not branches), so the sums take one LDS
            // round trip rather than one per key.
            float wt[max_books];
            uint32_t pv[max_books];
#pragma unroll
            for (int t = 0; t < max_books; ++t)
            {
                wt[t] = weights[t];
                pv[t] = values[t * (HW / 2) + j];
            }
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int t = 0; t < max_books; ++t)
            {
                const float a0 = __builtin_fmaf(__uint_as_float(pv[t] << 16), wt[t], s0);
                const float a1 = __builtin_fmaf(__uint_as_float(pv[t] & 0xffff0000u), wt[t], s1);
                s0 = t < time ? a0 : s0;
                s1 = t < time ? a1 : s1;
            }
            // The one block merged into the empty state (src/scalar/attention.cpp:86-101).
            float total, n0, n1;
            if (is_finite(maximum))
            {
                total = sum + 0.0f;
                n0 = s0 + 0.0f;
                n1 = s1 + 0.0f;
            }
            else
            {
                const float running_maximum = -__builtin_inff();
                const float factor = original_exp(-__builtin_fabsf(maximum - running_maximum));
                const float old_scale = running_maximum > maximum ? 1.0f : factor;
                const float new_scale = running_maximum > maximum ? factor : 1.0f;
                total = __builtin_fmaf(sum, new_scale, 0.0f * old_scale);
                n0 = __builtin_fmaf(s0, new_scale, 0.0f * old_scale);
                n1 = __builtin_fmaf(s1, new_scale, 0.0f * old_scale);
            }
            const float reciprocal = 1.0f / total;
            *reinterpret_cast<uint32_t*>(row + head * HW + 2 * j) =
                float_to_bf16(n0 * reciprocal) | (uint32_t(float_to_bf16(n1 * reciprocal)) << 16);
            return;
        }
    }
#pragma unroll 1
    for (int k = 0; k < count; ++k)
    {
        const int head = head_of(k);
        const float* query = query_of(head);
        const float* keys = keys_of(head);
        const uint32_t* values = values_of(head);
        float* weights = reinterpret_cast<float*>(values_of(head) + max_books * HW / 2);
        // 3. Scores (src/scalar/attention.cpp:27-35): lane t dots key row t with
        //    the query in ascending coordinates; operands requested `ahead`
        //    chunks before their use.
        float score = -__builtin_inff();
        if (lane < time)
        {
            const float4* q4 = reinterpret_cast<const float4*>(query);
            const float4* k4 = reinterpret_cast<const float4*>(keys + lane * key_stride);
            constexpr int chunks = HW / 4, ahead = 4;
            float4 qs[ahead], ks[ahead];
#pragma unroll
            for (int c = 0; c < ahead; ++c)
            {
                qs[c] = q4[c];
                ks[c] = k4[c];
            }
            float dot = 0.0f;
#pragma unroll
            for (int c = 0; c < chunks; ++c)
            {
                float4 qc = qs[c % ahead];
                const float4 kc = ks[c % ahead];
                if (c + ahead < chunks)
                {
                    qs[c % ahead] = q4[c + ahead];
                    ks[c % ahead] = k4[c + ahead];
                }
                in_vgprs(qc);
                dot = __builtin_fmaf(qc.x, kc.x, dot);
                dot = __builtin_fmaf(qc.y, kc.y, dot);
                dot = __builtin_fmaf(qc.z, kc.z, dot);
                dot = __builtin_fmaf(qc.w, kc.w, dot);
            }
            score = dot * scale;
        }
        const float maximum = group_max<wave>(score);
        float e = 0.0f;
        if (lane < time)
        {
            e = original_exp(score - maximum);
        }
        const float sum = tree_sum<wave>(e);
        weights[lane] = e;
        asm volatile("" ::: "memory");
        wait_shared_memory();
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");

        // 4. Value sums in ascending positions (src/scalar/attention.cpp:41-52).
        float s[per_lane];
#pragma unroll
        for (int i = 0; i < per_lane; ++i)
        {
            s[i] = 0.0f;
        }
        // Every key's weight and value word requested before the first is
        // used; steps past `time` are dropped by selects.
        float wt[max_books];
        uint32_t pv[max_books];
#pragma unroll
        for (int t = 0; t < max_books; ++t)
        {
            wt[t] = weights[t];
            pv[t] = values[t * (HW / 2) + (per_lane * lane) / 2];
        }
#pragma unroll
        for (int t = 0; t < max_books; ++t)
        {
            const float w = wt[t];
            const uint32_t pw = pv[t];
            if constexpr (per_lane == 2)
            {
                const float a0 = __builtin_fmaf(__uint_as_float(pw << 16), w, s[0]);
                const float a1 = __builtin_fmaf(__uint_as_float(pw & 0xffff0000u), w, s[1]);
                s[0] = t < time ? a0 : s[0];
                s[1] = t < time ? a1 : s[1];
            }
            else
            {
                const uint32_t v = (lane & 1) ? (pw >> 16) : (pw & 0xffffu);
                const float a0 = __builtin_fmaf(__uint_as_float(v << 16), w, s[0]);
                s[0] = t < time ? a0 : s[0];
            }
        }

        // 5. The one block merged into the empty state (src/scalar/attention.cpp:86-101).
        const float block_maximum = uniform(maximum), block_total = uniform(sum);
        float total, numerator[per_lane];
        if (is_finite(block_maximum))
        {
            // The finite original_exp(-88) scales the zero totals: each result is
            // the block's value plus +0.
            total = block_total + 0.0f;
#pragma unroll
            for (int i = 0; i < per_lane; ++i)
            {
                numerator[i] = s[i] + 0.0f;
            }
        }
        else
        {
            const float running_maximum = -__builtin_inff();
            const float factor = original_exp(-__builtin_fabsf(block_maximum - running_maximum));
            const float old_scale = running_maximum > block_maximum ? 1.0f : factor;
            const float new_scale = running_maximum > block_maximum ? factor : 1.0f;
            total = __builtin_fmaf(block_total, new_scale, 0.0f * old_scale);
#pragma unroll
            for (int i = 0; i < per_lane; ++i)
            {
                numerator[i] = __builtin_fmaf(s[i], new_scale, 0.0f * old_scale);
            }
        }
        const float reciprocal = 1.0f / total;
        if constexpr (per_lane == 2)
        {
            *reinterpret_cast<uint32_t*>(row + head * HW + 2 * lane) =
                float_to_bf16(numerator[0] * reciprocal) | (uint32_t(float_to_bf16(numerator[1] * reciprocal)) << 16);
        }
        else
        {
            row[head * HW + lane] = float_to_bf16(numerator[0] * reciprocal);
        }
    }
}

// One tile of R output rows of a projection for M lanes (decode.hip
// fused_linear_kernel). R is tile_rows, or narrow_rows for a K of 2 *
// frame_waves blocks: each half-wave then holds one whole block of 32 rows,
// block `warp` in lanes 0-31 and block `warp + frame_waves` in lanes 32-63, so
// every wave keeps its weights in registers for all lanes. A narrow tile t is
// rows [32 (t % 2), 32 (t % 2) + 32) of the 64-row weight tile t / 2.
template <int V, In I, Out O, int HW = 0, int R = tile_rows>
__device__ __noinline__ JOB void project_tile(constant_ptr<Projection> job, int position, int M, int tile, Exchange exchange,
                                          uint32_t* error, uint8_t* lds, constant_ptr<BookAttention> book_job = nullptr,
                                          int book_lane = 0, uint32_t previous_epoch = 0)
{
    const Exchange x{uint32_t(uniform(int(exchange.epoch))), uniform(exchange.abort)};
    lds = in_lds(lds);
    Projection p;
    p.w.values = uniform(job->w.values);
    p.w.scales = uniform(job->w.scales);
    p.w.bias = uniform(job->w.bias);
    p.w.K = uniform(job->w.K);
    p.w.N = uniform(job->w.N);
    p.x = uniform(job->x);
    p.gain = uniform(job->gain);
    p.beta = uniform(job->beta);
    p.embeddings = uniform(job->embeddings);
    p.alphabet = uniform(job->alphabet);
    p.books = uniform(job->books);
    p.book = uniform(job->book);
    p.tokens = uniform(job->tokens);
    p.token_stride = uniform(job->token_stride);
    p.token_words = uniform(job->token_words);
    p.token_book_words = uniform(job->token_book_words);
    previous_epoch = uint32_t(uniform(int(previous_epoch)));
    p.prefix_in = uniform(job->prefix_in);
    p.prefix_out = uniform(job->prefix_out);
    p.residual = uniform(job->residual);
    p.residual_row = uniform(job->residual_row);
    p.y = uniform(job->y);
    p.position = uniform(position);
    p.rotations = uniform(job->rotations);
    p.width = uniform(job->width);
    p.head_width = uniform(job->head_width);
    BookAttention book;
    if constexpr (I == In::attention)
    {
        book.qkv = uniform(book_job->qkv);
        book.book_words = uniform(book_job->book_words);
        book.time = uniform(book_job->time);
        book.lane = uniform(book_lane);
        book.scale = uniform(book_job->scale);
    }
    M = uniform(M);
    tile = uniform(tile);
    error = uniform(error);
    constexpr int K = wave * V, blocks = K / 256;
    constexpr bool narrow = R == narrow_rows;
    static_assert(R == tile_rows || (narrow && blocks == 2 * frame_waves), "narrow tiles hold two blocks per wave");
    constexpr int waves_per_block = blocks >= frame_waves ? 1 : frame_waves / blocks;
    constexpr int wave_segments = segments / waves_per_block;
    constexpr int rounds = narrow ? 1 : blocks > frame_waves ? blocks / frame_waves : 1;
    // Lanes one at a time whenever the weights fit registers for all of them.
    constexpr bool pipelined = rounds == 1;
    static_assert(I != In::attention || (pipelined && book_attention_fits<V, HW>),
                  "attention rows: one lane at a time, at most two heads per wave");
    // A pipelined tile spreads each input row over its first SW waves
    // (row_ops.hpp), Vw = V / SW values per lane; the other waves only keep
    // the row's barriers.
    constexpr int SW = spread_waves<V>;
    constexpr int Vw = V / SW;
    constexpr bool spread = pipelined && V % SW == 0 &&
                            (I == In::words || I == In::words_norm || I == In::attention);
    // Barriers inside the spread LayerNorm (one exchange of the wave sums) and
    // BF8L (one exchange of block maxima when a block spans waves).
    constexpr int spread_barriers =
        (I == In::words_norm && SW > 1 ? 1 : 0) + (Vw > 0 && 256 / Vw > wave ? 1 : 0);
    static_assert(I != In::attention || spread, "attention rows are spread");
    int8_t* q = reinterpret_cast<int8_t*>(lds);
    float* scales = reinterpret_cast<float*>(lds + max_lanes * K);
    int* dots = reinterpret_cast<int*>(lds + max_lanes * K + max_lanes * blocks * 4);
    const int lane = threadIdx.x % wave;
    const int warp = __builtin_amdgcn_readfirstlane(int(threadIdx.x / wave));
    const int N = int(p.w.N);

    // 1. Weight loads first, then the chain constants and the residual word.
    const int first_block = narrow ? warp + (lane / narrow_rows) * frame_waves
                            : rounds > 1 ? warp : warp / waves_per_block;
    const int first_segment = rounds > 1 || narrow ? 0 : (warp % waves_per_block) * wave_segments;
    uint4 w[wave_segments];
    {
        const int8_t* base = narrow ? p.w.values + tile_offset(tile / 2, first_block, 0, blocks) +
                                          ((tile % 2) * narrow_rows + lane % narrow_rows) * 16
                                    : p.w.values + tile_offset(tile, first_block, first_segment, blocks) + lane * 16;
#pragma unroll
        for (int s = 0; s < wave_segments; ++s)
        {
            w[s] = load16(base + s * tile_rows * 16);
        }
    }
    const int pair = threadIdx.x % (R / 2), column = threadIdx.x / (R / 2);
    const int n0 = tile * R + 2 * pair;
    const float2 bias = load_float2(p.w.bias + n0);
    const float bias0 = bias.x, bias1 = bias.y;
    // A fixed residual row (the codebook position row) is known before any wait.
    uint32_t fixed_residual = 0;
    if constexpr (O == Out::residual_row)
    {
        fixed_residual = *global(reinterpret_cast<const uint32_t*>(p.residual_row + n0));
    }
    float ws0[blocks], ws1[blocks];
#pragma unroll
    for (int b = 0; b < blocks; ++b)
    {
        const float2 s = load_float2(p.w.scales + std::size_t(b) * N + n0);
        ws0[b] = s.x;
        ws1[b] = s.y;
    }
    const std::size_t out_word = (std::size_t(column) * N + n0) / 2;
    // Rotary (cosine, sine) of this pair at the position, before any wait.
    uint32_t rotation = 0;
    if constexpr (O == Out::qkv)
    {
        if (p.rotations && n0 < 2 * p.width)
        {
            rotation = *global(reinterpret_cast<const uint32_t*>(
                p.rotations + std::size_t(p.position) * p.head_width + n0 % p.head_width));
        }
    }
    // LayerNorm constants of this lane's input values, before any wait.
    uint16_t norm_gain[V], norm_bias[V], spread_gain[Vw > 0 ? Vw : 1], spread_bias[Vw > 0 ? Vw : 1];
    if constexpr (I == In::words_norm && spread)
    {
        if (warp < SW)
        {
            load_global_row<Vw>(p.gain + (warp * wave + lane) * Vw, spread_gain);
            load_global_row<Vw>(p.beta + (warp * wave + lane) * Vw, spread_bias);
        }
    }
    else if constexpr (I == In::words_norm)
    {
        if (warp < M)
        {
            load_values<V>(p.gain + lane * V, norm_gain);
            load_values<V>(p.beta + lane * V, norm_bias);
        }
    }
    float* norm_exchange = reinterpret_cast<float*>(lds + projection_exchange<V>()); // [2 * frame_waves]
    uint32_t* scale_exchange = reinterpret_cast<uint32_t*>(norm_exchange + 2 * frame_waves); // [frame_waves]
    lds_barrier(); // the previous job's readers of LDS are done

    // Phases 2-4 for lanes [m0, m1). Pipelined tiles run them one lane at a
    // time in lane order, so lane m's output is published as soon as lane m's
    // input is in, without waiting for the later lanes (whose inputs come
    // later when they follow the range decoder's stream order); the weights
    // stay in registers across the lanes, so this needs a single round.
    const auto run_lanes = [&](int m0, int m1)
    {
        word residual_seen = 0;
        bool residual_requested = false;
        uint16_t prefix_row[I == In::embed_accumulate ? V : 1]; // tile 0's accumulated embedding row
        // 2. Inputs, quantised into LDS: a spread row is taken, normalised and
        //    quantised by all waves together; an attention row is computed by
        //    them (wave w takes heads w, w + frame_waves, ...) and then
        //    quantised the same way; other inputs take one row per wave (wave
        //    m reads lane m).
        if constexpr (I == In::attention)
        {
            constexpr int heads = K / HW;
            float* regions = reinterpret_cast<float*>(lds + projection_lds<V>());
            uint16_t* row = reinterpret_cast<uint16_t*>(regions + heads * book_head_floats<HW>);
            if (warp < heads)
            {
                constexpr int per_wave = (heads + frame_waves - 1) / frame_waves;
                residual_requested = O == Out::residual_words && column == m0;
                wave_book_heads<HW, per_wave>(book.qkv, book.book_words, book.time, K, book.scale, m0, warp,
                                              (heads - warp + frame_waves - 1) / frame_waves, x, regions, row,
                                              residual_requested ? p.residual + out_word : nullptr, residual_seen);
            }
            lds_barrier();
            if (warp < SW)
            {
                uint16_t v[Vw];
                load_row<Vw>(row + (warp * wave + lane) * Vw, v);
                bf8l_spread<Vw, SW>(v, warp, q + m0 * K, scales + m0 * blocks, error, scale_exchange);
            }
            else
            {
#pragma unroll
                for (int i = 0; i < spread_barriers; ++i)
                {
                    lds_barrier();
                }
            }
        }
        else if constexpr (spread)
        {
            if (warp < SW)
            {
                uint16_t v[Vw];
                if constexpr (Vw % 8 == 0)
                {
                    take_row<Vw>(p.x, std::size_t(m0) * K + (warp * wave + lane) * Vw, x, v);
                }
                else
                {
                    take_values<Vw>(p.x, std::size_t(m0) * K + (warp * wave + lane) * Vw, x, v);
                }
                if constexpr (I == In::words_norm)
                {
                    layer_norm_spread<Vw, SW>(v, spread_gain, spread_bias, warp, norm_exchange);
                }
                bf8l_spread<Vw, SW>(v, warp, q + m0 * K, scales + m0 * blocks, error, scale_exchange);
            }
            else
            {
#pragma unroll
                for (int i = 0; i < spread_barriers; ++i)
                {
                    lds_barrier();
                }
            }
        }
        else if (warp >= m0 && warp < m1)
        {
            uint16_t v[V];
            const std::size_t first = std::size_t(warp) * K + lane * V;
            if constexpr (I == In::words || I == In::words_norm)
            {
                take_row<V>(p.x, first, x, v);
                if constexpr (I == In::words_norm)
                {
                    layer_norm_values<V>(v, norm_gain, norm_bias);
                }
            }
            else if constexpr (I == In::embed_sum)
            {
                // src/common/cpu_transformer.tpp:205-224: copy book 0, add later books in order.
                // The previous step's tokens: from `tokens` at a launch's first
                // step (written before the launch), else from that step's
                // token words.
                const uint16_t* t = p.tokens + std::size_t(warp) * p.token_stride;
                // Lane b holds book b's token: polled from its token word (all
                // books' at once), or read from `tokens`.
                uint32_t previous = 0;
                {
                    const int b = lane < p.books ? lane : p.books - 1;
                    if (previous_epoch != 0)
                    {
                        previous = take(p.token_words + std::size_t(b) * p.token_book_words, warp,
                                        Exchange{previous_epoch, x.abort});
                    }
                    else
                    {
                        previous = *global(t + b);
                    }
                }
                const auto token_of = [&](int b)
                { return min(int(__builtin_amdgcn_readlane(previous, b) & 0xffff), p.alphabet - 1); };
                const int t0 = token_of(0);
                load_global_row<V>(p.embeddings + std::size_t(t0) * K + lane * V, v);
                // Book b's row is requested `ahead` books before it is added,
                // so the sum waits for about one row's latency rather than one
                // per book. Every request is made (past the last book it
                // repeats the last book's row, never added), so the requests
                // outstanding at each add do not depend on the book count.
                constexpr int ahead = 4, chunks = V / 4;
                static_assert(V % 4 == 0, "rows in 8-byte chunks");
                unsigned long long raw[ahead][chunks];
                const auto request = [&](int b, unsigned long long (&row)[chunks])
                {
                    const int book = b < p.books ? b : p.books - 1;
                    const auto* src = reinterpret_cast<const unsigned long long*>(
                        p.embeddings + (std::size_t(book) * p.alphabet + token_of(book)) * K + lane * V);
#pragma unroll
                    for (int c = 0; c < chunks; ++c)
                    {
                        row[c] = *global(src + c);
                    }
                };
#pragma unroll
                for (int i = 0; i < ahead; ++i)
                {
                    request(1 + i, raw[i]);
                }
                // Groups of `ahead` books, slot k holding book b0 + k.
                for (int b0 = 1; b0 < p.books; b0 += ahead)
                {
#pragma unroll
                    for (int k = 0; k < ahead; ++k)
                    {
                        if (b0 + k < p.books)
                        {
#pragma unroll
                            for (int i = 0; i < V; ++i)
                            {
                                const uint16_t e = uint16_t(raw[k][i / 4] >> (16 * (i % 4)));
                                v[i] = float_to_bf16(bf16_to_float(v[i]) + bf16_to_float(e));
                            }
                        }
                        request(b0 + k + ahead, raw[k]);
                    }
                }
            }
            else
            {
                const int token = min(int(take(p.token_words, warp, x) & 0xffffu), p.alphabet - 1);
                load_global_row<V>(p.embeddings + (std::size_t(p.book) * p.alphabet + token) * K + lane * V, v);
                if (p.prefix_in)
                {
                    uint16_t prev[V];
                    take_row<V>(p.prefix_in, first, x, prev);
#pragma unroll
                    for (int i = 0; i < V; ++i)
                    {
                        v[i] = float_to_bf16(bf16_to_float(prev[i]) + bf16_to_float(v[i]));
                    }
                }
                if (tile == 0)
                {
#pragma unroll
                    for (int i = 0; i < V; ++i)
                    {
                        prefix_row[i] = v[i];
                    }
                }
            }
            bf8l_lane<V>(v, lane, q + warp * K, scales + warp * blocks, error);
        }
        // The residual rows come from an earlier job than the inputs just read, so
        // requesting them now costs no wait of its own.
        if constexpr (O == Out::residual_words)
        {
            if (column >= m0 && column < m1 && !residual_requested)
            {
                residual_seen = peek(p.residual, out_word);
            }
        }
        lds_barrier();

        // 3. Exact partial dots.
#pragma unroll
        for (int r = 0; r < rounds; ++r)
        {
            const int b = rounds > 1 ? warp + r * frame_waves : first_block;
            if (r > 0)
            {
                const int8_t* base = p.w.values + tile_offset(tile, b, 0, blocks) + lane * 16;
#pragma unroll
                for (int s = 0; s < wave_segments; ++s)
                {
                    w[s] = load16(base + s * tile_rows * 16);
                }
            }
            const int slot = b * waves_per_block + (rounds > 1 || narrow ? 0 : warp % waves_per_block);
            for (int m = m0; m < m1; ++m)
            {
                // Four independent accumulators: the block dot is an exact
                // integer (|dot| < 2^24), so their order does not matter,
                // and the chain is a quarter as long.
                const uint4* xq = reinterpret_cast<const uint4*>(q + m * K + b * 256 + first_segment * 16);
                uint4 u[wave_segments];
#pragma unroll
                for (int s = 0; s < wave_segments; ++s)
                {
                    u[s] = xq[s];
                }
                int part[4] = {0, 0, 0, 0};
#pragma unroll
                for (int s = 0; s < wave_segments; ++s)
                {
                    part[0] = __builtin_amdgcn_sdot4(int(w[s].x), int(u[s].x), part[0], false);
                    part[1] = __builtin_amdgcn_sdot4(int(w[s].y), int(u[s].y), part[1], false);
                    part[2] = __builtin_amdgcn_sdot4(int(w[s].z), int(u[s].z), part[2], false);
                    part[3] = __builtin_amdgcn_sdot4(int(w[s].w), int(u[s].w), part[3], false);
                }
                dots[(slot * max_lanes + m) * R + lane % R] = (part[0] + part[1]) + (part[2] + part[3]);
            }
        }
        lds_barrier();

        // 4. Ordered chain per (row pair, column), then the output.
        if (column >= m0 && column < m1)
        {
            const int m = column;
            // Every partial dot and scale is requested before the first is
            // used: one LDS round trip for the chain instead of one per few
            // blocks.
            int2 part[blocks][waves_per_block];
            float as[blocks];
#pragma unroll
            for (int b = 0; b < blocks; ++b)
            {
#pragma unroll
                for (int s = 0; s < waves_per_block; ++s)
                {
                    part[b][s] = *reinterpret_cast<const int2*>(dots + ((b * waves_per_block + s) * max_lanes + m) * R +
                                                                2 * pair);
                }
                as[b] = scales[m * blocks + b];
            }
            __builtin_amdgcn_sched_barrier(0);
            float sum0 = 0.0f, sum1 = 0.0f;
#pragma unroll
            for (int b = 0; b < blocks; ++b)
            {
                int d0 = 0, d1 = 0;
#pragma unroll
                for (int s = 0; s < waves_per_block; ++s)
                {
                    d0 += part[b][s].x;
                    d1 += part[b][s].y;
                }
                const float scale0 = ws0[b] * as[b];
                const float scale1 = ws1[b] * as[b];
                sum0 = __builtin_fmaf(float(d0), scale0, sum0);
                sum1 = __builtin_fmaf(float(d1), scale1, sum1);
            }
            uint16_t y0 = float_to_bf16(sum0 + bias0);
            uint16_t y1 = float_to_bf16(sum1 + bias1);
            if constexpr (O == Out::residual_words)
            {
                const uint32_t r = settle(p.residual, out_word, residual_seen, x);
                y0 = float_to_bf16(bf16_to_float(uint16_t(r & 0xffff)) + bf16_to_float(y0));
                y1 = float_to_bf16(bf16_to_float(uint16_t(r >> 16)) + bf16_to_float(y1));
            }
            else if constexpr (O == Out::residual_row)
            {
                y0 = float_to_bf16(bf16_to_float(uint16_t(fixed_residual & 0xffff)) + bf16_to_float(y0));
                y1 = float_to_bf16(bf16_to_float(uint16_t(fixed_residual >> 16)) + bf16_to_float(y1));
            }
            else if constexpr (O == Out::gelu)
            {
                y0 = gelu_bf16(y0);
                y1 = gelu_bf16(y1);
            }
            else if constexpr (O == Out::qkv)
            {
                const int width = p.width;
                if (n0 < 2 * width && p.rotations)
                {
                    // rotate() of step_ops.hpp on the prefetched coefficients.
                    const float cosine = bf16_to_float(uint16_t(rotation & 0xffff)), sine = bf16_to_float(uint16_t(rotation >> 16));
                    const float re = bf16_to_float(y0), im = bf16_to_float(y1);
                    const float im_sine = im * sine;
                    const float re_sine = re * sine;
                    y0 = float_to_bf16(__builtin_fmaf(re, cosine, -im_sine));
                    y1 = float_to_bf16(__builtin_fmaf(im, cosine, re_sine));
                }
            }
            publish(p.y, out_word, y0 | (uint32_t(y1) << 16), x.epoch);
        }
        // The accumulated embedding row for the next book's prefix job goes
        // out only now: published before the dots, its stores would hold up
        // this tile's output (a later wait for any load also waits for the
        // stores issued before it), and the next prefix job reads it a whole
        // book later.
        if constexpr (I == In::embed_accumulate)
        {
            if (tile == 0 && warp >= m0 && warp < m1)
            {
                give_row<V>(p.prefix_out, std::size_t(warp) * K + lane * V, x, prefix_row);
            }
        }
    };
    if constexpr (pipelined)
    {
        if constexpr (I == In::attention)
        {
            run_lanes(book.lane, book.lane + 1);
        }
        else
        {
            for (int m = 0; m < M; ++m)
            {
                run_lanes(m, m + 1);
            }
        }
    }
    else
    {
        run_lanes(0, M);
    }
}

// ------------------------------------------------------------------ attention job

struct Attend
{
    int heads = 0, width = 0;
    float scale = 0.0f;
    int time = 0; // keys 0 .. time-1
    // Temporal: rows before time-1 from the cache (this layer, lane 0, row 0),
    // row time-1 from `qkv`, then stored into the cache. Codebook (keys ==
    // null): row t from the qkv words of book t at qkv + t*book_words.
    uint16_t* keys = nullptr;
    uint16_t* values = nullptr;
    long long lane_stride = 0;
    const word* qkv = nullptr;
    std::size_t book_words = 0;
    word* out = nullptr;
    // Temporal, split in halves: the block records of blocks 8-15, item i's
    // block b field f at word ((i * 8) + b - 8) * (2 + HW) + f.
    word* records = nullptr;
};

// This lane's value columns of the 64 rows of a block: with two columns per
// lane a word per row; with one, two rows per word (row 2i in the low half,
// row 2i + 1 in the high half, loaded there directly), which halves the
// registers. get(tt) returns the row's word with column c in bits 16c..16c+15.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
template <int per_lane> struct BlockValues;
template <> struct BlockValues<2>
{
    uint32_t word[64];
    __device__ __forceinline__ void set(int tt, uint32_t w)
    {
        word[tt] = w;
    }
    __device__ __forceinline__ uint32_t get(int tt) const
    {
        return word[tt];
    }
};
template <> struct BlockValues<1>
{
    u16x2 half[32];
    __device__ __forceinline__ void set(int tt, uint32_t w)
    {
        half[tt / 2][tt % 2] = uint16_t(w);
    }
    __device__ __forceinline__ uint32_t get(int tt) const
    {
        const uint32_t pair = __builtin_bit_cast(uint32_t, half[tt / 2]);
        return tt % 2 == 0 ? pair & 0xffffu : pair >> 16;
    }
};

// A temporal query of more than frame_waves blocks on one workgroup gives
// each wave a second block. With 64-wide heads the cached key and value rows
// of those blocks (16 KiB each) are requested into LDS at the job's start,
// as whole-row 16-byte loads, beside the job's other LDS.
template <int HW> constexpr bool stage_second_blocks = HW == 64;
template <int HW> constexpr int second_block_bytes = 2 * 64 * HW * 2; // key rows, then value rows

template <int HW> constexpr int attend_base_lds()
{
    // partial records, the fp32 query, staged exchanged rows (key words then
    // value words), codebook keys in fp32, each wave's block weights
    return (max_blocks * (2 + HW) + HW + max_books * HW + max_books * staged_key_stride<HW> + frame_waves * 64) * 4;
}
template <int HW> constexpr int attend_lds()
{
    static_assert(attend_base_lds<HW>() % 16 == 0, "second blocks 16-byte aligned");
    return attend_base_lds<HW>() + (stage_second_blocks<HW> ? frame_waves * second_block_bytes<HW> : 0);
}

// Position (16-byte slot) of chunk c of row r of a block staged by
// stage_block: rows in groups of 64 / chunks_per_row per 1 KiB request, the
// chunks of row r rotated by r, so that lanes reading "their" row at the same
// chunk fall on distinct banks.
template <int HW> __device__ __forceinline__ int staged_slot(int r, int c)
{
    constexpr int chunks = HW * 2 / 16, rows = 64 / chunks;
    return 64 * (r / rows) + chunks * (r % rows) + (c + r) % chunks;
}

// Requests the cached rows [start, start + count) (count <= 64, each of HW
// BF16 values) of `rows` into `to` (LDS) in staged_slot order, one 16-byte
// chunk per lane and 1 KiB per request: lanes 8 g .. 8 g + 7 of request j
// read row (64 / chunks) j + g whole. The data lands when the wave's vector
// memory counter says so.
template <int HW>
__device__ __forceinline__ void stage_block(const uint16_t* rows, std::size_t stride, int start, int count,
                                            uint8_t* to, int lane)
{
    constexpr int chunks = HW * 2 / 16, per_request = 64 / chunks, requests = 64 / per_request;
#pragma unroll
    for (int j = 0; j < requests; ++j)
    {
        const int r = j * per_request + lane / chunks, slot = lane % chunks;
        const int c = ((slot - r) % chunks + chunks) % chunks;
        if (r < count)
        {
            __builtin_amdgcn_global_load_lds(global(rows + std::size_t(start + r) * stride + c * 8),
                                             (__attribute__((address_space(3))) void*)(to + j * 1024), 16, 0, 0);
        }
    }
}

// One (lane, head) query over all its keys (decode.hip attention_step_kernel).
// The rows that come through exchange words (the current position's, or every
// codebook row) and the query are staged in LDS first, so the block loops read
// only the cache and LDS.
// A temporal query may be split in halves over two workgroups: half 1 takes
// blocks 8-15 (when there are more than 8) and hands their records to half 0
// in exchange words; half 0 takes blocks 0-7, then those records, and merges
// every block in ascending order as one workgroup would. Each half stores the
// cache rows of its own blocks, so a row is read back through the L2 that
// wrote it. `half` -1 is one workgroup for all blocks.
template <int HW>
__device__ __noinline__ JOB void attend_item(constant_ptr<Attend> job, int keys, int item, int half, Exchange exchange,
                                         uint8_t* lds)
{
    const Exchange x{uint32_t(uniform(int(exchange.epoch))), uniform(exchange.abort)};
    lds = in_lds(lds);
    Attend a;
    a.heads = uniform(job->heads);
    a.width = uniform(job->width);
    a.scale = uniform(job->scale);
    a.time = uniform(keys);
    a.keys = uniform(job->keys);
    a.values = uniform(job->values);
    a.lane_stride = uniform(job->lane_stride);
    a.qkv = uniform(job->qkv);
    a.book_words = uniform(job->book_words);
    a.out = uniform(job->out);
    a.records = uniform(job->records);
    item = uniform(item);
    half = uniform(half);
    constexpr int per_lane = HW / 64; // value columns per lane (adjacent)
    constexpr int row_words = HW;     // staged row: HW/2 key words, then HW/2 value words
    constexpr int key_stride = staged_key_stride<HW>;
    float* partial = reinterpret_cast<float*>(lds);        // [blocks][2 + HW]
    float* query = partial + max_blocks * (2 + HW);         // [HW]
    uint32_t* staged = reinterpret_cast<uint32_t*>(query + HW); // [max_books][row_words]
    float* staged_keys = reinterpret_cast<float*>(staged + max_books * row_words); // [max_books][key_stride]
    float* weights = staged_keys + max_books * key_stride; // [frame_waves][64]
    const int m = item / a.heads, head = item % a.heads;
    const int lane = threadIdx.x % wave;
    const int warp = __builtin_amdgcn_readfirstlane(int(threadIdx.x / wave));
    const int time = a.time;
    const int blocks = (time + 63) / 64;
    const bool round_values = time > 64;
    const int width = a.width;
    const bool temporal = a.keys != nullptr;
    if (half == 1 && (!temporal || blocks <= frame_waves))
    {
        return; // half 0 has every block
    }
    // This workgroup's blocks [first_block, end_block) and whether it stores
    // this step's cache row (the owner of the row's block).
    const int first_block = half == 1 ? frame_waves : 0;
    const int end_block = half == 0 ? min(blocks, frame_waves) : blocks;
    const bool stores_row = half < 0 || half == ((time - 1) / 64 >= frame_waves ? 1 : 0);
    const int cached = temporal ? time - 1 : 0; // rows 0..cached-1 come from the cache
    const int exchanged = time - cached;        // the rest from words (1, or time <= max_books)
    const std::size_t row_values = 3 * std::size_t(width);
    const std::size_t q_value = std::size_t(m) * row_values + head * HW;
    const auto row_words_of = [&](int t) -> const word*
    { return temporal ? a.qkv : a.qkv + std::size_t(t) * a.book_words; };
    const uint16_t* k = temporal ? a.keys + std::size_t(m) * a.lane_stride + head * HW : nullptr;
    const uint16_t* v = temporal ? a.values + std::size_t(m) * a.lane_stride + head * HW : nullptr;

    // Key words and value words of one 64-key block: lane l holds key row
    // block*64 + l, and this lane's value columns of row block*64 + tt
    // (BlockValues).
    // Temporal attention reads every row but the last (time - 1) from the
    // cache; book attention reads all its rows (time <= max_books) from the
    // exchange.
    uint32_t key[HW / 2];
    BlockValues<per_lane> value;
    // Cache rows need nothing from this step: requested before any wait.
    const auto load_cached = [&](int block)
    {
        const int start = block * 64;
        const int count = time - start < 64 ? time - start : 64;
        const int t = start + lane;
        if (lane < count && t < cached)
        {
            const uint16_t* row = k + std::size_t(t) * width;
#pragma unroll
            for (int c = 0; c < HW / 8; ++c)
            {
                const uint4 u = load16(row + 8 * c);
                key[4 * c] = u.x;
                key[4 * c + 1] = u.y;
                key[4 * c + 2] = u.z;
                key[4 * c + 3] = u.w;
            }
        }
        if constexpr (per_lane == 2)
        {
#pragma unroll
            for (int tt = 0; tt < 64; ++tt)
            {
                const int row = start + tt;
                if (tt < count && row < cached)
                {
                    value.word[tt] = *global(reinterpret_cast<const uint32_t*>(v + std::size_t(row) * width + 2 * lane));
                }
            }
        }
        else
        {
            // Every row is requested, rows past the cached ones as the last
            // cached row (or row 0), whose values are never used: a request
            // under a per-row branch would be waited for before the next one,
            // as each row's value joins another in a register.
            const int last = cached > 0 ? cached - 1 : 0;
#pragma unroll
            for (int tt = 0; tt < 64; ++tt)
            {
                const int row = start + tt < cached ? start + tt : last;
                value.half[tt / 2][tt % 2] = *global(v + std::size_t(row) * width + lane);
            }
        }
    };
    if (temporal && first_block + warp < end_block)
    {
        load_cached(first_block + warp);
    }

    // 1. Stage the query and the exchanged rows: word i of the query is i < HW/2;
    //    then row r's key words, then its value words. The query and the keys
    //    of codebook rows are stored as fp32 (exact: BF16 is the top half of
    //    an fp32), so the score chains read operands without unpacking them.
    lds_barrier(); // the previous job's readers of LDS are done
    // The wave's second block, when it has one, is requested into LDS now.
    const int second_block = first_block + warp + frame_waves;
    const bool second_staged = stage_second_blocks<HW> && temporal && half < 0 && second_block < end_block;
    uint8_t* const second = lds + attend_base_lds<HW>() + warp * second_block_bytes<HW>;
    if (second_staged)
    {
        const int start = second_block * 64;
        const int count = min(time - start, 64), from_cache = min(cached - start, count);
        stage_block<HW>(k, width, start, from_cache, second, lane);
        stage_block<HW>(v, width, start, from_cache, second + second_block_bytes<HW> / 2, lane);
    }
    {
        constexpr int per_thread = (HW / 2 + max_books * row_words + frame_threads - 1) / frame_threads;
        const int total = HW / 2 + exchanged * row_words;
        uint32_t got[per_thread];
        const auto address = [&](int i) -> const word*
        {
            int index = int(threadIdx.x) + i * frame_threads;
            index = index < total ? index : total - 1;
            if (index < HW / 2)
            {
                return row_words_of(time - 1) + q_value / 2 + index;
            }
            const int r = (index - HW / 2) / row_words, c = (index - HW / 2) % row_words;
            const std::size_t value0 = q_value + (c < HW / 2 ? width : 2 * width);
            return row_words_of(cached + r) + value0 / 2 + c % (HW / 2);
        };
        take_words<per_thread>(address, x, got);
#pragma unroll
        for (int i = 0; i < per_thread; ++i)
        {
            const int index = int(threadIdx.x) + i * frame_threads;
            const float2 pair = make_float2(__uint_as_float(got[i] << 16), __uint_as_float(got[i] & 0xffff0000u));
            if (index < HW / 2)
            {
                reinterpret_cast<float2*>(query)[index] = pair;
            }
            else if (index < total)
            {
                const int r = (index - HW / 2) / row_words, c = (index - HW / 2) % row_words;
                if (!temporal && c < HW / 2)
                {
                    reinterpret_cast<float2*>(staged_keys + r * key_stride)[c] = pair;
                }
                else
                {
                    staged[index - HW / 2] = got[i];
                }
            }
        }
    }
    lds_barrier();
    // Temporal: this step's key and value row joins the cache, stored by the
    // workgroup that owns this (lane, head) in every step, so the later steps
    // of the launch read it back through the same L2.
    if (temporal && stores_row && threadIdx.x < row_words)
    {
        const int i = int(threadIdx.x);
        uint16_t* to = (i < HW / 2 ? a.keys : a.values) + std::size_t(m) * a.lane_stride + std::size_t(cached) * width +
                       head * HW + 2 * (i % (HW / 2));
        *global_out(reinterpret_cast<uint32_t*>(to)) = staged[i];
    }

    // The value word of staged row r for this lane's columns.
    const auto staged_value = [&](int r) -> uint32_t
    {
        const uint32_t pw = staged[r * row_words + HW / 2 + (per_lane * lane) / 2];
        return per_lane == 2 ? pw : ((lane & 1) ? (pw >> 16) : (pw & 0xffff));
    };
    if (!temporal)
    {
#pragma unroll
        for (int tt = 0; tt < max_books; ++tt)
        {
            if (tt < time)
            {
                value.set(tt, staged_value(tt));
            }
        }
    }

    // 2. Blocks of 64 keys: wave w owns blocks w, w + waves, ...
    float* block_weights = weights + warp * 64;
    float kept[2 + per_lane]; // the last block's maximum, total and value sums
    for (int block = first_block + warp; block < end_block; block += frame_waves)
    {
        if (block == second_block && second_staged)
        {
            // The cached rows requested at the start (staged_slot order).
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            const int start = block * 64;
            const int count = time - start < 64 ? time - start : 64;
            const int t = start + lane;
            if (lane < count && t < cached)
            {
#pragma unroll
                for (int c = 0; c < HW / 8; ++c)
                {
                    const uint4 u = *reinterpret_cast<const uint4*>(second + 16 * staged_slot<HW>(lane, c));
                    key[4 * c] = u.x;
                    key[4 * c + 1] = u.y;
                    key[4 * c + 2] = u.z;
                    key[4 * c + 3] = u.w;
                }
            }
            // Every row's slot is read (those past the requested rows hold
            // values that are never used).
            const uint8_t* values_in = second + second_block_bytes<HW> / 2;
            const int byte = 2 * per_lane * lane; // this lane's columns within a row
#pragma unroll
            for (int tt = 0; tt < 64; ++tt)
            {
                const uint8_t* at = values_in + 16 * staged_slot<HW>(tt, byte / 16) + byte % 16;
                if constexpr (per_lane == 2)
                {
                    value.word[tt] = *reinterpret_cast<const uint32_t*>(at);
                }
                else
                {
                    value.half[tt / 2][tt % 2] = *reinterpret_cast<const uint16_t*>(at);
                }
            }
        }
        else if (block != first_block + warp)
        {
            load_cached(block);
        }
        const int start = block * 64;
        const int count = time - start < 64 ? time - start : 64;
        const int t = start + lane;
        if (temporal && lane < count && t >= cached)
        {
            const uint4* row = reinterpret_cast<const uint4*>(staged + (t - cached) * row_words);
#pragma unroll
            for (int c = 0; c < HW / 8; ++c)
            {
                const uint4 u = row[c];
                key[4 * c] = u.x;
                key[4 * c + 1] = u.y;
                key[4 * c + 2] = u.z;
                key[4 * c + 3] = u.w;
            }
        }
        float score = -__builtin_inff();
        if (lane < count)
        {
            // Ascending coordinates (src/scalar/attention.cpp:27-35).
            float dot = 0.0f;
            // LDS operands are requested `ahead` chunks before their use: one
            // chunk's FMAs take far less time than an LDS round trip.
            const float4* q4 = reinterpret_cast<const float4*>(query);
            if (temporal)
            {
                // Key words in registers (cache rows and the staged last row).
                constexpr int chunks = HW / 4, ahead = 2;
                float4 qs[ahead];
#pragma unroll
                for (int c = 0; c < ahead; ++c)
                {
                    qs[c] = q4[c];
                }
#pragma unroll
                for (int c = 0; c < chunks; ++c)
                {
                    float4 qc = qs[c % ahead];
                    if (c + ahead < chunks)
                    {
                        qs[c % ahead] = q4[c + ahead];
                    }
                    in_vgprs(qc);
                    const float q[4] = {qc.x, qc.y, qc.z, qc.w};
#pragma unroll
                    for (int i = 0; i < 2; ++i)
                    {
                        const uint32_t kw = key[2 * c + i];
                        dot = __builtin_fmaf(q[2 * i], __uint_as_float(kw << 16), dot);
                        dot = __builtin_fmaf(q[2 * i + 1], __uint_as_float(kw & 0xffff0000u), dot);
                    }
                }
            }
            else
            {
                // Codebook keys in fp32 in LDS, row t per lane.
                const float4* row = reinterpret_cast<const float4*>(staged_keys + t * key_stride);
                constexpr int chunks = HW / 4, ahead = 4;
                float4 qs[ahead], ks[ahead];
#pragma unroll
                for (int c = 0; c < ahead; ++c)
                {
                    qs[c] = q4[c];
                    ks[c] = row[c];
                }
#pragma unroll
                for (int c = 0; c < chunks; ++c)
                {
                    float4 qc = qs[c % ahead];
                    const float4 kc = ks[c % ahead];
                    if (c + ahead < chunks)
                    {
                        qs[c % ahead] = q4[c + ahead];
                        ks[c % ahead] = row[c + ahead];
                    }
                    in_vgprs(qc);
                    dot = __builtin_fmaf(qc.x, kc.x, dot);
                    dot = __builtin_fmaf(qc.y, kc.y, dot);
                    dot = __builtin_fmaf(qc.z, kc.z, dot);
                    dot = __builtin_fmaf(qc.w, kc.w, dot);
                }
            }
            score = dot * a.scale;
        }
        const float maximum = group_max<wave>(score);
        float e = 0.0f;
        if (lane < count)
        {
            e = original_exp(score - maximum);
        }
        const float sum = tree_sum<wave>(e);
        block_weights[lane] = e;
        wait_shared_memory();
        // Ascending positions (src/scalar/attention.cpp:41-52); the staged
        // last row of a temporal history comes last.
        const int from_values = temporal ? (cached - start < count ? cached - start : count) : count;
        // The weights needed, all requested before the first is used.
        float4 w4[16];
#pragma unroll
        for (int t4 = 0; t4 < 16; ++t4)
        {
            if (4 * t4 < from_values)
            {
                w4[t4] = reinterpret_cast<const float4*>(block_weights)[t4];
            }
        }
        float s0 = 0.0f, s1 = 0.0f;
        const auto accumulate = [&](uint32_t vw, float w)
        {
            s0 = __builtin_fmaf(__uint_as_float(vw << 16), w, s0);
            if (per_lane == 2)
            {
                s1 = __builtin_fmaf(__uint_as_float(vw & 0xffff0000u), w, s1);
            }
        };
#pragma unroll
        for (int t4 = 0; t4 < 16; ++t4)
        {
            if (4 * t4 >= from_values)
            {
                break;
            }
            in_vgprs(w4[t4]);
            const float w[4] = {w4[t4].x, w4[t4].y, w4[t4].z, w4[t4].w};
            if (4 * t4 + 4 <= from_values)
            {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                {
                    accumulate(value.get(4 * t4 + i), w[i]);
                }
            }
            else if (4 * t4 < from_values)
            {
#pragma unroll
                for (int i = 0; i < 3; ++i)
                {
                    if (4 * t4 + i < from_values)
                    {
                        accumulate(value.get(4 * t4 + i), w[i]);
                    }
                }
            }
        }
        if (from_values < count)
        {
            accumulate(staged_value(0), block_weights[count - 1]);
        }
        // The block's record: lane 0's maximum and total, this lane's value sums.
        kept[0] = uniform(maximum);
        kept[1] = uniform(sum);
        kept[2] = round_values ? round_bf16(s0) : s0;
        if constexpr (per_lane == 2)
        {
            kept[3] = round_values ? round_bf16(s1) : s1;
        }
        if (blocks > 1)
        {
            float* record = partial + std::size_t(block) * (2 + HW);
            if (lane == 0)
            {
                record[0] = kept[0];
                record[1] = kept[1];
            }
#pragma unroll
            for (int i = 0; i < per_lane; ++i)
            {
                record[2 + per_lane * lane + i] = kept[2 + i];
            }
            __builtin_amdgcn_wave_barrier();
        }
    }
    // A single block (every codebook query, and temporal ones up to 64 keys)
    // is wave 0's own: its record stays in registers, with no barrier.
    if (blocks > 1)
    {
        lds_barrier();
    }
    if (half >= 0 && blocks > frame_waves)
    {
        constexpr int record_floats = 2 + HW;
        const int count = (blocks - frame_waves) * record_floats;
        word* const records = a.records + std::size_t(item) * frame_waves * record_floats;
        float* const second = partial + std::size_t(frame_waves) * record_floats;
        if (half == 1)
        {
            // Hand the records of blocks 8.. over, and stop.
            for (int i = int(threadIdx.x); i < count; i += frame_threads)
            {
                publish(records, i, __float_as_uint(second[i]), x.epoch);
            }
            return;
        }
        constexpr int per_thread = (frame_waves * record_floats + frame_threads - 1) / frame_threads;
        uint32_t got[per_thread];
        take_words<per_thread>(
            [&](int i) -> const word*
            {
                const int index = int(threadIdx.x) + i * frame_threads;
                return records + (index < count ? index : count - 1);
            },
            x, got);
#pragma unroll
        for (int i = 0; i < per_thread; ++i)
        {
            const int index = int(threadIdx.x) + i * frame_threads;
            if (index < count)
            {
                second[index] = __uint_as_float(got[i]);
            }
        }
        lds_barrier();
    }
    if (warp != 0)
    {
        return;
    }
    // 3. Ordered merge of the blocks (src/scalar/attention.cpp:86-101).
    float numerator[per_lane];
#pragma unroll
    for (int i = 0; i < per_lane; ++i)
    {
        numerator[i] = 0.0f;
    }
    float running_maximum = -__builtin_inff(), total = 0.0f;
    const auto merge = [&](float maximum, float block_total, const float* values)
    {
        const float difference = maximum - running_maximum;
        const float factor = original_exp(-__builtin_fabsf(difference));
        const float old_scale = running_maximum > maximum ? 1.0f : factor;
        const float new_scale = running_maximum > maximum ? factor : 1.0f;
        const float old_total = total * old_scale;
        total = __builtin_fmaf(block_total, new_scale, old_total);
#pragma unroll
        for (int i = 0; i < per_lane; ++i)
        {
            const float old = numerator[i] * old_scale;
            numerator[i] = __builtin_fmaf(values[i], new_scale, old);
        }
        running_maximum = running_maximum < maximum ? maximum : running_maximum;
    };
    if (blocks == 1 && is_finite(kept[0]))
    {
        // Merging one block with a finite maximum into the empty state scales
        // the zero totals by the finite original_exp(-88): each result is the
        // block's value plus +0.
        total = kept[1] + 0.0f;
#pragma unroll
        for (int i = 0; i < per_lane; ++i)
        {
            numerator[i] = kept[2 + i] + 0.0f;
        }
    }
    else if (blocks == 1)
    {
        merge(kept[0], kept[1], kept + 2);
    }
    else
    {
        // Lane b holds block b's maximum and total. Without NaN maxima the
        // running maximum before each block is a scan with the recurrence's
        // own update, so every block's factors come at once (block b's from
        // lane b) and the ordered chain left is two fmas per block, with the
        // factors broadcast from their lanes; with a NaN the plain loop runs.
        const float maximum = lane < blocks ? partial[std::size_t(lane) * (2 + HW)] : -__builtin_inff();
        const float block_total = lane < blocks ? partial[std::size_t(lane) * (2 + HW) + 1] : 0.0f;
        if (__any(__builtin_isnan(maximum)))
        {
            for (int b = 0; b < blocks; ++b)
            {
                const float* record = partial + std::size_t(b) * (2 + HW);
                merge(record[0], record[1], record + 2 + per_lane * lane);
            }
        }
        else
        {
            const float running = previous_lane(running_max_scan(maximum), -__builtin_inff());
            const float factor = original_exp(-__builtin_fabsf(maximum - running));
            const float old_scale = running > maximum ? 1.0f : factor;
            const float new_scale = running > maximum ? factor : 1.0f;
            float sums[max_blocks][per_lane];
#pragma unroll
            for (int b = 0; b < max_blocks; ++b)
            {
                if (b < blocks)
                {
#pragma unroll
                    for (int i = 0; i < per_lane; ++i)
                    {
                        sums[b][i] = partial[std::size_t(b) * (2 + HW) + 2 + per_lane * lane + i];
                    }
                }
            }
#pragma unroll
            for (int b = 0; b < max_blocks; ++b)
            {
                if (b < blocks)
                {
                    const float os = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(old_scale), b));
                    const float ns = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(new_scale), b));
                    const float bt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(block_total), b));
                    total = __builtin_fmaf(bt, ns, total * os);
#pragma unroll
                    for (int i = 0; i < per_lane; ++i)
                    {
                        numerator[i] = __builtin_fmaf(sums[b][i], ns, numerator[i] * os);
                    }
                }
            }
        }
    }
    const float reciprocal = 1.0f / total;
    const std::size_t at = std::size_t(m) * width + head * HW + per_lane * lane;
    if constexpr (per_lane == 2)
    {
        const uint32_t packed = float_to_bf16(numerator[0] * reciprocal) |
                                (uint32_t(float_to_bf16(numerator[1] * reciprocal)) << 16);
        publish(a.out, at / 2, packed, x.epoch);
    }
    else
    {
        const uint32_t mine = float_to_bf16(numerator[0] * reciprocal);
        const uint32_t other = lane_swap1(mine);
        if ((lane & 1) == 0)
        {
            publish(a.out, at / 2, mine | (other << 16), x.epoch);
        }
    }
}

// ------------------------------------------------------------------ conditioning job

// Book 0's codebook input: bf16(LayerNorm(x) + positions[0]) for every lane,
// one wave per lane (decode.hip layer_norm_add_kernel).
template <int V>
__device__ __noinline__ JOB void condition_rows(const word* in, const uint16_t* gain, const uint16_t* bias,
                                            const uint16_t* add_row, word* out, int M, Exchange exchange)
{
    const Exchange x{uint32_t(uniform(int(exchange.epoch))), uniform(exchange.abort)};
    in = uniform(in);
    gain = uniform(gain);
    bias = uniform(bias);
    add_row = uniform(add_row);
    out = uniform(out);
    M = uniform(M);
    constexpr int width = wave * V;
    const int lane = threadIdx.x % wave;
    const int row = __builtin_amdgcn_readfirstlane(int(threadIdx.x / wave));
    if (row >= M)
    {
        return;
    }
    // Constants first: the input is the last thing to arrive.
    uint16_t g[V], b[V], p[V];
    load_global_row<V>(gain + lane * V, g);
    load_global_row<V>(bias + lane * V, b);
    load_global_row<V>(add_row + lane * V, p);
    uint16_t v[V];
    take_row<V>(in, std::size_t(row) * width + lane * V, x, v);
    layer_norm_values<V>(v, g, b);
#pragma unroll
    for (int i = 0; i < V; ++i)
    {
        v[i] = float_to_bf16(bf16_to_float(v[i]) + bf16_to_float(p[i]));
    }
    give_row<V>(out, std::size_t(row) * width + lane * V, x, v);
}

// ------------------------------------------------------------------ sampling job

constexpr int window = 256;
constexpr int draw_lds =
    max_lanes * 1024 * 4 + max_lanes * 1024 * 2 + max_lanes * 64 * 2 + window + 3 * max_lanes * 4 + 3 * frame_waves * 4;

struct Draw
{
    int book = 0, books = 0;
    const word* logits = nullptr; // [lanes][1024] in words
    word* token_words = nullptr;  // one per lane
    uint16_t* current = nullptr;
    uint16_t* tokens = nullptr;
    const int* row_base = nullptr;
    int step = 0, step_stride = 0;
    const uint16_t* known = nullptr;
    uint16_t* distributions = nullptr;
    uint16_t* splits = nullptr; // known tokens: each token's ten Q15 splits at [row][16]
    const uint8_t* payload = nullptr;
    unsigned long long payload_bytes = 0;
};

// Inputs of book 0's conditioning rows (condition_rows).
struct Condition
{
    const word* in = nullptr;
    const uint16_t* gain = nullptr;
    const uint16_t* bias = nullptr;
    const uint16_t* positions = nullptr;
    word* out = nullptr;
};

// Where each job's descriptor sits in the job table: projections (the temporal
// embedding, 4 per temporal layer, then per book its prefix, 4 per codebook
// layer and its head), attention jobs (temporal layers, then (book, layer)),
// the fused codebook attention per (book, layer), one draw per book and the
// conditioning rows; each part 256-byte aligned.
struct JobTable
{
    int TL, CL, C;
    __host__ __device__ JobTable(int temporal_layers, int codebook_layers, int books)
        : TL(temporal_layers), CL(codebook_layers), C(books)
    {
    }
    __host__ __device__ static constexpr std::size_t align(std::size_t n)
    {
        return (n + 255) / 256 * 256;
    }
    __host__ __device__ int embed() const
    {
        return 0;
    }
    __host__ __device__ int temporal(int layer, int op) const
    {
        return 1 + 4 * layer + op;
    }
    __host__ __device__ int prefix(int book) const
    {
        return 1 + 4 * TL + book * (4 * CL + 2);
    }
    __host__ __device__ int codebook(int book, int layer, int op) const
    {
        return prefix(book) + 1 + 4 * layer + op;
    }
    __host__ __device__ int head(int book) const
    {
        return prefix(book) + 4 * CL + 1;
    }
    __host__ __device__ int projections() const
    {
        return prefix(C);
    }
    __host__ __device__ int attend(bool temporal_layer, int book, int layer) const
    {
        return temporal_layer ? layer : TL + book * CL + layer;
    }
    __host__ __device__ std::size_t projection_offset(int index) const
    {
        return std::size_t(index) * sizeof(Projection);
    }
    __host__ __device__ std::size_t attend_offset(int index) const
    {
        return align(std::size_t(projections()) * sizeof(Projection)) + std::size_t(index) * sizeof(Attend);
    }
    __host__ __device__ std::size_t book_offset(int index) const
    {
        return attend_offset(TL + C * CL) + std::size_t(index) * sizeof(BookAttention);
    }
    __host__ __device__ std::size_t draw_offset(int book) const
    {
        return align(book_offset(C * CL)) + std::size_t(book) * sizeof(Draw);
    }
    __host__ __device__ std::size_t condition_offset() const
    {
        return align(draw_offset(C));
    }
    __host__ __device__ std::size_t bytes() const
    {
        return align(condition_offset() + sizeof(Condition));
    }
};

// Lane 0's softmax (src/common/probability.cpp:96-122) and subtree masses
// (build_masses' nodes) by all waves: its logits arrive first, as the lanes
// follow the range decoder's stream order, while the other waves would wait.
// Wave w takes symbols [128w, 128w + 128), two per lane, so each wave's trees
// are the reference's pair trees over its part and the waves' results join as
// the trees' top levels. `exchange` is 3 * frame_waves words of LDS. Returns
// (in wave 0) whether every probability is finite and non-negative.
__device__ __forceinline__ bool first_lane_masses(const word* logits, uint16_t* distributions, bool decoding,
                                                  const Exchange& x, uint32_t* error, float* nodes, uint16_t* leaves,
                                                  float* exchange)
{
    const int lane = threadIdx.x % wave, warp = __builtin_amdgcn_readfirstlane(int(threadIdx.x / wave));
    const int position = warp * wave + lane; // symbols 2 * position and 2 * position + 1
    uint16_t v[2];
    take_values<2>(logits, std::size_t(position) * 2, x, v);
    float maximum = -__builtin_inff();
    bool finite = true;
#pragma unroll
    for (int k = 0; k < 2; ++k)
    {
        const float value = bf16_to_float(v[k]);
        finite = finite && is_finite(value);
        maximum = maximum < value ? value : maximum;
    }
    if (!finite)
    {
        error[0] = 1u;
    }
    maximum = group_max<wave>(maximum);
    if (lane == 0)
    {
        exchange[warp] = maximum;
    }
    lds_barrier();
#pragma unroll
    for (int w = 0; w < frame_waves; ++w)
    {
        const float m = exchange[w];
        maximum = maximum < m ? m : maximum;
    }
    float e[2], sum[2];
#pragma unroll
    for (int k = 0; k < 2; ++k)
    {
        e[k] = original_exp(bf16_to_float(v[k]) - maximum);
        sum[k] = e[k];
    }
    const float part = tree_sum<wave>(register_tree<2>(sum));
    if (lane == 0)
    {
        exchange[frame_waves + warp] = part;
    }
    lds_barrier();
    float parts[frame_waves];
#pragma unroll
    for (int w = 0; w < frame_waves; ++w)
    {
        parts[w] = exchange[frame_waves + w];
    }
    // probability_sum ends with add(+0, S) (src/format/categorical.cpp:44-74).
    const float total = flushed_add(0.0f, flushed_tree<frame_waves>(parts));
    const float reciprocal = 1.0f / total;
    float prob[2];
#pragma unroll
    for (int k = 0; k < 2; ++k)
    {
        v[k] = float_to_bf16(e[k] * reciprocal);
        prob[k] = bf16_to_float(v[k]);
    }
    const uint32_t pair = v[0] | (uint32_t(v[1]) << 16);
    if (distributions)
    {
        *global_out(reinterpret_cast<uint32_t*>(distributions + 2 * position)) = pair;
    }
    if (!decoding)
    {
        return true;
    }
    *reinterpret_cast<uint32_t*>(leaves + 2 * position) = pair;
    bool valid = is_finite(prob[0]) && prob[0] >= 0.0f && is_finite(prob[1]) && prob[1] >= 0.0f;
    // Node n covers 1024 >> floor(log2 n) symbols; after the butterfly at
    // stride s a lane's value covers 4s symbols from 2 * position.
    float m = flushed_add(flush(prob[0]), flush(prob[1]));
    nodes[512 + position] = m;
    const auto store = [&](int s) {
        if (position % (2 * s) == 0)
        {
            nodes[256 / s + position / (2 * s)] = m;
        }
    };
    m = butterfly_ftz_add<1>(m);
    store(1);
    m = butterfly_ftz_add<2>(m);
    store(2);
    m = butterfly_ftz_add<4>(m);
    store(4);
    m = butterfly_ftz_add<8>(m);
    store(8);
    m = butterfly_ftz_add<16>(m);
    store(16);
    m = butterfly_ftz_add<32>(m);
    store(32); // node 8 + warp
    if (lane == 0)
    {
        exchange[2 * frame_waves + warp] = __all(valid) ? 1.0f : 0.0f;
    }
    lds_barrier();
    if (warp != 0)
    {
        return true;
    }
    // Nodes 1..7 from the waves' nodes 8..15.
    float level[frame_waves];
    valid = true;
#pragma unroll
    for (int w = 0; w < frame_waves; ++w)
    {
        level[w] = nodes[frame_waves + w];
        valid = valid && exchange[2 * frame_waves + w] != 0.0f;
    }
#pragma unroll
    for (int width = frame_waves / 2; width >= 1; width /= 2)
    {
#pragma unroll
        for (int i = 0; i < width; ++i)
        {
            level[i] = flushed_add(level[2 * i], level[2 * i + 1]);
            if (lane == 0)
            {
                nodes[width + i] = level[i];
            }
        }
    }
    return valid;
}

// A flag in LDS that hands data in LDS from one wave of the workgroup to
// another. LDS performs one wave's accesses in order, so the writer's data is
// in once its own LDS accesses are done (lgkmcnt(0)), and the reader's later
// LDS reads follow its read of the flag. A release or acquire at workgroup
// scope would also wait for the wave's global stores (such as the tokens just
// published), which this hand-off does not need.
__device__ __forceinline__ void raise_lds_flag(int* flag)
{
    asm volatile("" ::: "memory");
    wait_shared_memory();
    __hip_atomic_store((__attribute__((address_space(3))) int*)(flag), 1, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_WORKGROUP);
    asm volatile("" ::: "memory");
}
__device__ __forceinline__ bool lds_flag_raised(int* flag)
{
    const int v = __hip_atomic_load((__attribute__((address_space(3))) int*)(flag), __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_WORKGROUP);
    asm volatile("" ::: "memory");
    return v != 0;
}

// Stores the compiler does not track, for a wave that never reads back what
// it stored: for a tracked store the compiler waits for the acknowledgement
// (s_waitcnt vmcnt(0)) before it reuses the store's data registers, while the
// decoding wave's next symbol needs nothing from memory. The vector-memory
// counter retires in issue order, so stores left out of the compiler's count
// only ever make its own waits longer, never shorter. sc1 is the cache policy
// of an agent-scope atomic store (the exchange words are polled with
// agent-scope loads).
__device__ __forceinline__ void untracked_store_u16(uint16_t* p, uint32_t value)
{
    asm volatile("global_store_short %0, %1, off" ::"v"(p), "v"(value) : "memory");
}
__device__ __forceinline__ void untracked_publish(word* w, std::size_t index, uint32_t payload, uint32_t epoch)
{
    const word value = (word(epoch) << 32) | payload;
    asm volatile("global_store_dwordx2 %0, %1, off sc1" ::"v"(w + index), "v"(value) : "memory");
}

// Softmax, masses and top decisions per lane: lane 0's by all waves
// (first_lane_masses), every later lane's by one wave; wave 0 decodes the
// lanes' symbols in stream order with the decoder held in `state` (LDS)
// (decode.hip sample_kernel), each once its lane's masses are released.
__device__ __noinline__ JOB void draw_tokens(constant_ptr<Draw> job, int step, int M, DecoderState* state, Exchange exchange,
                                         uint32_t* error, uint8_t* lds)
{
    const Exchange x{uint32_t(uniform(int(exchange.epoch))), uniform(exchange.abort)};
    lds = in_lds(lds);
    state = reinterpret_cast<DecoderState*>(in_lds(reinterpret_cast<uint8_t*>(state)));
    Draw a;
    a.book = uniform(job->book);
    a.books = uniform(job->books);
    a.logits = uniform(job->logits);
    a.token_words = uniform(job->token_words);
    a.current = uniform(job->current);
    a.tokens = uniform(job->tokens);
    a.row_base = uniform(job->row_base);
    a.step = uniform(step);
    a.step_stride = uniform(job->step_stride);
    a.known = uniform(job->known);
    a.distributions = uniform(job->distributions);
    a.splits = uniform(job->splits);
    a.payload = uniform(job->payload);
    a.payload_bytes = uniform(std::size_t(job->payload_bytes));
    M = uniform(M);
    error = uniform(error);
    float* nodes = reinterpret_cast<float*>(lds);                                         // [8][1024]
    uint16_t* leaves = reinterpret_cast<uint16_t*>(lds + max_lanes * 1024 * 4);           // [8][1024]
    uint16_t* top = reinterpret_cast<uint16_t*>(lds + max_lanes * 1024 * 6);              // [8][64]
    uint8_t* bytes = lds + max_lanes * (1024 * 6 + 128);                                  // [window]
    int* valid = reinterpret_cast<int*>(lds + max_lanes * (1024 * 6 + 128) + window);     // [8]
    int* rows = valid + max_lanes;                                                 // [8]
    int* ready = rows + max_lanes;                                                  // [8]
    float* partials = reinterpret_cast<float*>(ready + max_lanes);                  // [3 * waves]
    const int lane = threadIdx.x % wave, warp = __builtin_amdgcn_readfirstlane(int(threadIdx.x / wave));
    const bool active = warp < M;
    const bool decoding = a.known == nullptr;
    // Known tokens with splits: the masses are built as for decoding, and each
    // token's path splits are taken from them instead of a decode.
    const bool splitting = !decoding && a.splits != nullptr;
    int row = 0;
    if (active)
    {
        row = *global(a.row_base + warp) + a.step * a.step_stride + a.book;
    }
    lds_barrier(); // the previous job's readers of LDS are done; `state` is current
    if (threadIdx.x < max_lanes)
    {
        ready[threadIdx.x] = 0;
    }
    lds_barrier();
    // Wave 0 decodes, so it stages the payload window itself (zeros past the end).
    const unsigned long long base_offset = decoding ? state->offset : 0;
    if (warp == 0)
    {
        uint32_t four = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            const unsigned long long at = base_offset + uint32_t(lane * 4 + i);
            if (decoding && at < a.payload_bytes)
            {
                four |= uint32_t(*global(a.payload + at)) << (8 * i);
            }
        }
        reinterpret_cast<uint32_t*>(bytes)[lane] = four;
    }
    {
        const int first_row = *global(a.row_base) + a.step * a.step_stride + a.book;
        const bool ok = first_lane_masses(a.logits, a.distributions ? a.distributions + std::size_t(first_row) * 1024
                                                                    : nullptr,
                                          decoding || splitting, x, error, nodes, leaves, partials);
        if (warp == 0)
        {
            if (decoding)
            {
                wait_shared_memory();
                build_top_decisions(lane, Masses{nodes, leaves}, top);
            }
            // Lane 0's row, masses and decisions are in LDS: release them.
            if (lane == 0)
            {
                valid[0] = ok;
                rows[0] = first_row;
                raise_lds_flag(ready);
            }
        }
    }
    if (active && warp > 0)
    {
        uint16_t v[16];
        take_row<16>(a.logits, std::size_t(warp) * 1024 + lane * 16, x, v);
        if (lane == 0)
        {
            rows[warp] = row;
        }
        float maximum = -__builtin_inff();
        bool finite = true;
#pragma unroll
        for (int k = 0; k < 16; ++k)
        {
            const float value = bf16_to_float(v[k]);
            finite = finite && is_finite(value);
            maximum = maximum < value ? value : maximum;
        }
        if (!finite)
        {
            error[0] = 1u;
        }
        maximum = group_max<wave>(maximum);
        float e[16], leaves_sum[16];
#pragma unroll
        for (int k = 0; k < 16; ++k)
        {
            e[k] = original_exp(bf16_to_float(v[k]) - maximum);
            leaves_sum[k] = e[k];
        }
        const float total = row_sum<16>(leaves_sum);
        const float reciprocal = 1.0f / total;
        float prob[16];
#pragma unroll
        for (int k = 0; k < 16; ++k)
        {
            v[k] = float_to_bf16(e[k] * reciprocal);
            prob[k] = bf16_to_float(v[k]);
        }
        if (a.distributions)
        {
            store_row<16>(a.distributions + std::size_t(row) * 1024 + lane * 16, v);
        }
        if (decoding || splitting)
        {
            store_row<16>(leaves + warp * 1024 + lane * 16, v);
            const bool ok = build_masses(prob, lane, nodes + warp * 1024);
            wait_shared_memory();
            if (decoding)
            {
                build_top_decisions(lane, Masses{nodes + warp * 1024, leaves + warp * 1024}, top + warp * 64);
            }
            if (lane == 0)
            {
                valid[warp] = ok;
            }
        }
        // Lane `warp`'s row, masses and decisions are in LDS: release them to wave 0.
        if (lane == 0)
        {
            raise_lds_flag(ready + warp);
        }
    }
    if (warp != 0)
    {
        return;
    }
    // Wave 0 decodes the lanes' symbols in stream order (decode.hip sample_kernel),
    // each as soon as its lane's masses are in, and publishes each token at once,
    // so the next book of lane w can start while the later lanes are decoded.
    const auto output = [&](int w, int r, int token)
    {
        if (lane == 0)
        {
            untracked_publish(a.token_words, w, uint32_t(token), x.epoch);
            untracked_store_u16(a.current + std::size_t(w) * a.books + a.book, uint32_t(token));
            untracked_store_u16(a.tokens + r, uint32_t(token));
        }
    };
    const auto wait_for_lane = [&](int w)
    {
        while (!lds_flag_raised(ready + w))
        {
            __builtin_amdgcn_s_sleep(1);
        }
        return __builtin_amdgcn_readfirstlane(rows[w]);
    };
    // Two loops, so that the decoding one makes no global load whose
    // destination register a later lane's code reuses: the compiler would
    // then wait for all of the wave's memory accesses, the stores just made
    // included, at the start of every lane.
    if (!decoding)
    {
        for (int w = 0; w < M; ++w)
        {
            const int r = wait_for_lane(w);
            const int token = *global(a.known + r);
            output(w, r, token);
            if (splitting)
            {
                const uint16_t q = path_split(Masses{nodes + w * 1024, leaves + w * 1024}, token, lane);
                if (lane < 10)
                {
                    *global_out(a.splits + std::size_t(r) * 16 + lane) = q;
                }
            }
        }
        return;
    }
    DecoderState s = *state;
    const ByteWindow staged{bytes, window, base_offset, a.payload, a.payload_bytes};
    for (int w = 0; w < M; ++w)
    {
        const int r = wait_for_lane(w);
        if (!__builtin_amdgcn_readfirstlane(valid[w]))
        {
            s.failed = 1;
        }
        output(w, r, decode_symbol(top + w * 64, Masses{nodes + w * 1024, leaves + w * 1024}, s, staged));
    }
    if (lane == 0)
    {
        *state = s;
    }
}

// ------------------------------------------------------------------ the step

// V* = K/64 of the width, FFN and latent rows; HW the head width.
template <int VW, int VF, int VL, int HW> constexpr int frame_lds()
{
    return std::max({projection_lds<VW>() + book_attention_lds<VW, HW>(), projection_lds<VF>(), projection_lds<VL>(),
                     attend_lds<HW>(), draw_lds});
}

// How a frame step's jobs map onto `workers` workgroups (besides the sampler).
// Every kind of job owns a group of workgroups, one per tile when they fit.
// Two refinements, taken when the device holds their extra workgroups:
//  * fused: a codebook layer's attention (at most max_books keys) is computed
//    by its out-projection tiles, one workgroup per (tile, lane), instead of
//    by a job of its own followed by a hand-off;
//  * paired: qkv, up and down tiles (which take every lane in turn) get two
//    sets of workgroups that alternate between consecutive layers, so a
//    workgroup has two layers' time to finish its last lane and load the next
//    layer's weights before that layer's first input arrives.
// When the fused out tiles' extra workgroups do not fit, they are borrowed:
// the codebook layers' out tiles, attention included, run on the attention
// group, whose workgroups otherwise wait out the codebook stack (its
// attention being fused); the out group keeps the temporal out tiles.
struct FrameLayout
{
    bool fused = false, paired = false;
    bool borrowed = false; // fused codebook out tiles on the attention group
    bool split = false; // temporal queries in halves over two workgroups each
    // Down projections in tiles of narrow_rows output rows: their 64-row tiles
    // would hold more weight blocks than the waves can keep in registers, and a
    // tile that streams them in rounds takes all lanes at once. The embedding
    // job then runs on the prefix group's workgroups.
    bool narrow_down = false;
    int out_tiles = 0;  // tiles of an out job: one per lane when fused
    int down_tiles = 0; // tiles of a down job
    int workgroups = 0; // workers the layout asks for
};

__host__ __device__ inline FrameLayout frame_layout(int width, int heads, int ffn, int alphabet, int lanes, int workers)
{
    // At most two heads per wave (book_attention_fits).
    const bool fusable = heads <= max_book_heads_per_wave * frame_waves;
    const int w = width / tile_rows, f = ffn / tile_rows;
    FrameLayout l;
    l.narrow_down = ffn / 256 > frame_waves;
    l.down_tiles = l.narrow_down ? width / narrow_rows : w;
    // embed, qkv, attend, out, up, down, condition, prefix, head
    const int base = (l.narrow_down ? 0 : w) + 3 * w + lanes * heads + w + f + l.down_tiles + 1 + w +
                     alphabet / tile_rows;
    const int fused_extra = (lanes - 1) * w, paired_extra = 3 * w + f + l.down_tiles;
    if (fusable && base + fused_extra + paired_extra <= workers)
    {
        l.fused = l.paired = true;
    }
    else if (fusable && base + fused_extra <= workers)
    {
        l.fused = true;
    }
    else if (base + paired_extra <= workers)
    {
        l.paired = true;
    }
    if (fusable && !l.fused)
    {
        l.fused = l.borrowed = true;
    }
    l.out_tiles = l.fused && !l.borrowed ? lanes * w : w;
    l.workgroups = base + (l.fused && !l.borrowed ? fused_extra : 0) + (l.paired ? paired_extra : 0);
    if (l.workgroups + lanes * heads <= workers)
    {
        l.split = true;
        l.workgroups += lanes * heads;
    }
    return l;
}

template <int VW, int VF, int VL, int HW>
__global__ __launch_bounds__(frame_threads) void frame_kernel(const FrameArgs a)
{
    __shared__ __attribute__((aligned(16))) uint8_t lds[frame_lds<VW, VF, VL, HW>()];
    __shared__ DecoderState decoder;
    // The launch runs a.steps consecutive steps; each has its own epoch,
    // context position and step index.
    Exchange x{a.epoch, a.abort};
    int position = a.position, step_index = a.step;
    const Words L(a.width, a.ffn, a.latent, a.alphabet, a.books, a.temporal_layers, a.codebook_layers);
    const int M = a.lanes, G = int(gridDim.x), me = int(blockIdx.x);
    const int TL = a.temporal_layers, CL = a.codebook_layers, C = a.books, width = a.width;
    const int sampler = 0;
    if (me == sampler && threadIdx.x == 0 && a.known == nullptr)
    {
        decoder = *a.state;
    }
    // Workgroup 0 only samples. Every other workgroup runs one kind of job
    // (one function, so its code stays in the instruction cache), for every
    // layer and book: each kind owns a contiguous group of workgroups sized to
    // its tiles (scaled down if they do not all fit), tile t of a job going to
    // member t mod size. Consecutive jobs therefore run on different
    // workgroups, and each workgroup loads its next job's weights long before
    // that job's inputs exist.
    enum Kind
    {
        embed,
        qkv,
        attend,
        out,
        up,
        down,
        condition,
        prefix,
        head,
        kinds
    };
    const FrameLayout layout = frame_layout(width, a.heads, a.ffn, a.alphabet, M, G - 1);
    const auto sets = [&](int kind)
    { return layout.paired && (kind == Kind::qkv || kind == Kind::up || kind == Kind::down) ? 2 : 1; };
    // With layout.split, temporal queries go to two workgroups each
    // (attend_item's halves). Tiles [0, M*heads) are the second halves: a
    // workgroup runs its tiles in ascending order, so one that held both
    // halves of a query would hand the records over before it waits for them.
    const bool split_attention = layout.split;
    const int kind_tiles[kinds] = {width / tile_rows, 3 * width / tile_rows, (split_attention ? 2 : 1) * M * a.heads,
                                   layout.out_tiles, a.ffn / tile_rows, layout.down_tiles, 1, width / tile_rows,
                                   a.alphabet / tile_rows};
    // With narrow down tiles the embedding job runs on the prefix group (both
    // take width / tile_rows tiles): a prefix workgroup's embedding job of the
    // next step comes after its last prefix job of this step, in the order of
    // their inputs.
    const auto own_group = [&](int kind) { return !(layout.narrow_down && kind == Kind::embed); };
    int group_size[kinds], group_base[kinds];
    {
        const int workers = G - 1;
        int total = 0, owners = 0;
        for (int k = 0; k < kinds; ++k)
        {
            if (own_group(k))
            {
                total += kind_tiles[k] * sets(k);
                ++owners;
            }
        }
        int base = 1;
        for (int k = 0; k < kinds; ++k)
        {
            if (!own_group(k))
            {
                continue;
            }
            group_size[k] = total <= workers ? kind_tiles[k] * sets(k)
                                             : max(1, kind_tiles[k] * (workers - owners) / total);
            group_base[k] = base;
            base += group_size[k];
        }
        if (!own_group(Kind::embed))
        {
            group_size[Kind::embed] = group_size[Kind::prefix];
            group_base[Kind::embed] = group_base[Kind::prefix];
        }
    }
    // This workgroup's first tile of a job of `kind` (>= any tile count if
    // none); `parity` picks the set of a paired kind (the layer's parity).
    const auto first_tile = [&](int kind, int parity = 0)
    {
        const int none = G * max_lanes * 64;
        const int member = me - group_base[kind];
        if (member < 0 || member >= group_size[kind])
        {
            return none;
        }
        if (sets(kind) == 1)
        {
            return member;
        }
        return member / kind_tiles[kind] == parity ? member % kind_tiles[kind] : none;
    };
    // Distance between a workgroup's tiles of one job.
    const auto step = [&](int kind) { return group_size[kind] / sets(kind); };
    // Whether this workgroup takes tiles of `kind`. A job block is skipped whole
    // when it does not: building a job reads the model tables from memory, which
    // would put a round trip between every two jobs of the workgroup's own kind.
    const auto member = [&](int kind, int parity = 0) { return first_tile(kind, parity) < kind_tiles[kind]; };
    const JobTable T(TL, CL, C);
    const uint8_t* const jobs = static_cast<const uint8_t*>(a.jobs);
    const auto projection = [&](int index) { return constant<Projection>(jobs + T.projection_offset(index)); };
    const int width_tiles = width / tile_rows;

    // One stack layer: its four projections (table entries q + 0..3) and its
    // attention (table entry `att`, over `time` keys).
    const auto run_layer = [&](bool temporal, int q, int att, int time, int parity)
    {
        if (member(Kind::qkv, parity))
        {
            const auto p = projection(q);
            for (int t = first_tile(Kind::qkv, parity); t < 3 * width_tiles; t += step(Kind::qkv))
            {
                project_tile<VW, In::words_norm, Out::qkv>(p, position, M, t, x, a.error, lds);
            }
        }
        // Temporal attention is a job of its own; with the fused layout a
        // codebook layer's (at most max_books keys) is computed by each
        // out-projection tile itself.
        const bool fused = !temporal && layout.fused;
        if (!fused)
        {
            const auto attention = constant<Attend>(jobs + T.attend_offset(att));
            const int items = M * a.heads;
            for (int t = first_tile(Kind::attend); t < kind_tiles[Kind::attend]; t += group_size[Kind::attend])
            {
                const int half = !split_attention ? -1 : t < items ? 1 : 0;
                attend_item<HW>(attention, time, t % items, half, x, lds);
            }
        }
        if (fused && layout.borrowed)
        {
            // Tile t % width_tiles of lane t / width_tiles, on the attention group.
            if constexpr (book_attention_fits<VW, HW>)
            {
                if (member(Kind::attend))
                {
                    const auto p = projection(q + 1);
                    const auto book = constant<BookAttention>(jobs + T.book_offset(att - TL));
                    for (int t = first_tile(Kind::attend); t < M * width_tiles; t += group_size[Kind::attend])
                    {
                        project_tile<VW, In::attention, Out::residual_words, HW>(p, 0, M, t % width_tiles, x, a.error,
                                                                                 lds, book, t / width_tiles);
                    }
                }
            }
        }
        else if (member(Kind::out))
        {
            const auto p = projection(q + 1);
            if (!fused)
            {
                for (int t = first_tile(Kind::out); t < width_tiles; t += group_size[Kind::out])
                {
                    project_tile<VW, In::words, Out::residual_words>(p, 0, M, t, x, a.error, lds);
                }
            }
            else if constexpr (book_attention_fits<VW, HW>)
            {
                // One lane per workgroup: each stages its lane's earlier books
                // while it waits, and no lane waits for another's attention.
                const auto book = constant<BookAttention>(jobs + T.book_offset(att - TL));
                for (int t = first_tile(Kind::out); t < M * width_tiles; t += group_size[Kind::out])
                {
                    project_tile<VW, In::attention, Out::residual_words, HW>(p, 0, M, t % width_tiles, x, a.error, lds,
                                                                             book, t / width_tiles);
                }
            }
        }
        if (member(Kind::up, parity))
        {
            const auto p = projection(q + 2);
            for (int t = first_tile(Kind::up, parity); t < a.ffn / tile_rows; t += step(Kind::up))
            {
                project_tile<VW, In::words_norm, Out::gelu>(p, 0, M, t, x, a.error, lds);
            }
        }
        if (member(Kind::down, parity))
        {
            const auto p = projection(q + 3);
            for (int t = first_tile(Kind::down, parity); t < layout.down_tiles; t += step(Kind::down))
            {
                if (layout.narrow_down)
                {
                    if constexpr (VF * wave / 256 == 2 * frame_waves)
                    {
                        project_tile<VF, In::words, Out::residual_words, 0, narrow_rows>(p, 0, M, t, x, a.error, lds);
                    }
                }
                else
                {
                    project_tile<VF, In::words, Out::residual_words>(p, 0, M, t, x, a.error, lds);
                }
            }
        }
    };

    for (int s = 0; s < a.steps; ++s)
    {
        x.epoch = a.epoch + uint32_t(s);
        position = a.position + s;
        step_index = a.step + s;
        // Temporal stack: feedback embeddings of the previous frame, then layers.
        if (member(Kind::embed))
        {
            const auto p = projection(T.embed());
            const uint32_t previous_epoch = s > 0 ? x.epoch - 1u : 0u;
            for (int t = first_tile(Kind::embed); t < width_tiles; t += group_size[Kind::embed])
            {
                project_tile<VL, In::embed_sum, Out::plain>(p, 0, M, t, x, a.error, lds, nullptr, 0, previous_epoch);
            }
        }
        for (int l = 0; l < TL; ++l)
        {
            run_layer(true, T.temporal(l, 0), T.attend(true, 0, l), position + 1, l % 2);
        }
        // Book 0's input.
        if (first_tile(Kind::condition) == 0)
        {
            const auto c = constant<Condition>(jobs + T.condition_offset());
            condition_rows<VW>(c->in, c->gain, c->bias, c->positions, c->out, M, x);
        }
        for (int b = 0; b < C; ++b)
        {
            if (b > 0 && member(Kind::prefix))
            {
                const auto p = projection(T.prefix(b));
                for (int t = first_tile(Kind::prefix); t < width_tiles; t += group_size[Kind::prefix])
                {
                    project_tile<VL, In::embed_accumulate, Out::residual_row>(p, 0, M, t, x, a.error, lds);
                }
            }
            for (int l = 0; l < CL; ++l)
            {
                run_layer(false, T.codebook(b, l, 0), T.attend(false, b, l), b + 1, (TL + b * CL + l) % 2);
            }
            if (member(Kind::head))
            {
                const auto p = projection(T.head(b));
                for (int t = first_tile(Kind::head); t < a.alphabet / tile_rows; t += group_size[Kind::head])
                {
                    project_tile<VW, In::words_norm, Out::plain>(p, 0, M, t, x, a.error, lds);
                }
            }
            if (me == sampler)
            {
                draw_tokens(constant<Draw>(jobs + T.draw_offset(b)), step_index, M, &decoder, x, a.error, lds);
            }
        }
    }
    if (me == sampler && a.known == nullptr)
    {
        lds_barrier();
        if (threadIdx.x == 0)
        {
            *a.state = decoder;
            if (decoder.failed)
            {
                a.error[1] = 1u;
            }
        }
    }
}

// Workgroups of frame_kernel<VW, VF, VL, HW> that fit on the device at once,
// computed once per device.
template <int VW, int VF, int VL, int HW> int resident_workgroups()
{
    static std::array<std::atomic<int>, 64> resident{};
    int device = 0, units = 0, per_unit = 0;
    check_hip(hipGetDevice(&device), "hipGetDevice");
    require(device >= 0 && device < int(resident.size()), "frame step: device index out of range");
    if (const int known = resident[device].load(std::memory_order_relaxed))
    {
        return known;
    }
    check_hip(hipDeviceGetAttribute(&units, hipDeviceAttributeMultiprocessorCount, device), "hipDeviceGetAttribute");
    check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_unit, frame_kernel<VW, VF, VL, HW>, frame_threads, 0),
              "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    require(units > 0 && per_unit > 0, "frame step: kernel does not fit a compute unit");
    resident[device].store(units * per_unit, std::memory_order_relaxed);
    return units * per_unit;
}

template <int VW, int VF, int VL, int HW> FrameLaunch launch_frame(const FrameArgs& a, hipStream_t stream)
{
    const int resident = resident_workgroups<VW, VF, VL, HW>();
    // The workgroups of the richest layout the device holds (frame_kernel
    // derives the same layout from the grid), plus the sampler; when not even
    // the plain one fits, the groups shrink and workgroups take several tiles.
    const FrameLayout layout = frame_layout(a.width, a.heads, a.ffn, a.alphabet, a.lanes, resident - 1);
    const int grid = std::min(resident, layout.workgroups + 1);
    FrameArgs args = a;
    void* params[] = {&args};
    const void* kernel = reinterpret_cast<const void*>(frame_kernel<VW, VF, VL, HW>);
    if (a.plain_launch)
    {
        // Asked for by the session (for example to run under a profiler): the
        // grid fits the device at once, so on an otherwise idle device it is
        // co-resident; every wait of the kernel is bounded, so where it is not,
        // the step ends with the "stalled" error instead of hanging.
        check_hip(hipLaunchKernel(kernel, dim3(grid), dim3(frame_threads), params, 0, stream), "frame step launch");
        return FrameLaunch::requested_plain;
    }
    // Cooperative: every workgroup waits on others, so all must be resident at
    // once, also when several sessions share the device. A plain launch of the
    // same grid measured ~20 us less per step on an otherwise idle device, but
    // two concurrent sessions could then each hold part of the device and wait
    // on workgroups that cannot be placed.
    hipError_t status = hipLaunchCooperativeKernel(kernel, dim3(grid), dim3(frame_threads), params, 0, stream);
    if (status == hipErrorIllegalState)
    {
        // The device's cooperative-launch resources belong to one process at a
        // time, and another process holds them: the same grid goes out as a
        // plain launch, with the bounded waits above.
        (void)hipGetLastError();
        check_hip(hipLaunchKernel(kernel, dim3(grid), dim3(frame_threads), params, 0, stream), "frame step launch");
        return FrameLaunch::fallback_plain;
    }
    check_hip(status, "frame step launch");
    return FrameLaunch::cooperative;
}
} // namespace

std::vector<uint8_t> frame_job_table(const FrameArgs& a)
{
    const int TL = a.temporal_layers, CL = a.codebook_layers, C = a.books, width = a.width;
    require(a.words && a.model.linears && a.model.gain && a.model.bias, "frame job table: arguments");
    const Words L(a.width, a.ffn, a.latent, a.alphabet, C, TL, CL);
    const JobTable T(TL, CL, C);
    std::vector<uint8_t> table(T.bytes(), 0);
    word* const words = reinterpret_cast<word*>(a.words);
    const FrameModel& model = a.model;
    const auto put = [&](std::size_t offset, const auto& value)
    {
        require(offset + sizeof value <= table.size(), "frame job table: layout");
        std::memcpy(table.data() + offset, &value, sizeof value);
    };
    const auto linear = [&](bool temporal, int layer, int op) { return model.linears[(temporal ? 0 : 4 * TL) + 4 * layer + op]; };
    const auto norm = [&](bool temporal, int layer, bool mlp) { return (temporal ? 0 : 2 * TL + 1) + 2 * layer + (mlp ? 1 : 0); };
    // One stack layer (src/common/cpu_transformer.tpp:139-173): word ranges of
    // its input, qkv, attention, mid residual, hidden and output.
    const auto layer = [&](bool temporal, int l, int book, std::size_t in, std::size_t qkv, std::size_t att,
                           std::size_t mid, std::size_t hid, std::size_t output)
    {
        const int q = temporal ? T.temporal(l, 0) : T.codebook(book, l, 0);
        Projection p;
        p.w = linear(temporal, l, 0);
        p.x = words + in;
        p.gain = model.gain[norm(temporal, l, false)];
        p.beta = model.bias[norm(temporal, l, false)];
        p.y = words + qkv;
        p.width = width;
        p.head_width = a.head_width;
        if (temporal)
        {
            p.rotations = model.rotations;
        }
        put(T.projection_offset(q), p);
        Projection o;
        o.w = linear(temporal, l, 1);
        o.x = words + att;
        o.residual = words + in;
        o.y = words + mid;
        put(T.projection_offset(q + 1), o);
        Projection u;
        u.w = linear(temporal, l, 2);
        u.x = words + mid;
        u.gain = model.gain[norm(temporal, l, true)];
        u.beta = model.bias[norm(temporal, l, true)];
        u.y = words + hid;
        put(T.projection_offset(q + 2), u);
        Projection d;
        d.w = linear(temporal, l, 3);
        d.x = words + hid;
        d.residual = words + mid;
        d.y = words + output;
        put(T.projection_offset(q + 3), d);
        Attend at;
        at.heads = a.heads;
        at.width = width;
        at.scale = a.scale;
        at.out = words + att;
        if (temporal)
        {
            at.keys = a.keys + std::size_t(l) * a.extent * width;
            at.values = a.values + std::size_t(l) * a.extent * width;
            at.lane_stride = a.lane_stride;
            at.qkv = words + qkv;
            at.records = words + L.t_records(l);
        }
        else
        {
            at.qkv = words + L.c_qkv(0, l);
            at.book_words = L.book;
            BookAttention fused;
            fused.qkv = at.qkv;
            fused.book_words = at.book_words;
            fused.time = book + 1;
            fused.scale = a.scale;
            put(T.book_offset(book * CL + l), fused);
        }
        put(T.attend_offset(T.attend(temporal, book, l)), at);
    };

    Projection embed;
    embed.w = model.linears[4 * (TL + CL)];
    embed.embeddings = model.embeddings;
    embed.alphabet = a.alphabet;
    embed.books = C;
    embed.tokens = a.current;
    embed.token_stride = C;
    embed.token_words = words + L.c_token(0, CL);
    embed.token_book_words = L.book;
    embed.y = words + L.t_x(0);
    put(T.projection_offset(T.embed()), embed);
    for (int l = 0; l < TL; ++l)
    {
        layer(true, l, 0, L.t_x(l), L.t_qkv(l), L.t_att(l), L.t_mid(l), L.t_hid(l), L.t_x(l + 1));
    }
    Condition condition;
    condition.in = words + L.t_x(TL);
    condition.gain = model.gain[2 * TL];
    condition.bias = model.bias[2 * TL];
    condition.positions = model.positions;
    condition.out = words + L.c_x(0, 0);
    put(T.condition_offset(), condition);
    for (int b = 0; b < C; ++b)
    {
        if (b > 0)
        {
            Projection prefix;
            prefix.w = model.linears[4 * (TL + CL) + 1];
            prefix.embeddings = model.embeddings;
            prefix.alphabet = a.alphabet;
            prefix.book = b - 1;
            prefix.token_words = words + L.c_token(b - 1, CL);
            prefix.prefix_in = b > 1 ? words + L.c_prefix(b - 1) : nullptr;
            prefix.prefix_out = words + L.c_prefix(b);
            prefix.residual_row = model.positions + std::size_t(b) * width;
            prefix.y = words + L.c_x(b, 0);
            put(T.projection_offset(T.prefix(b)), prefix);
        }
        for (int l = 0; l < CL; ++l)
        {
            layer(false, l, b, L.c_x(b, l), L.c_qkv(b, l), L.c_att(b, l), L.c_mid(b, l), L.c_hid(b, l),
                  L.c_x(b, l + 1));
        }
        Projection head;
        head.w = model.linears[4 * (TL + CL) + 2];
        head.x = words + L.c_x(b, CL);
        head.gain = model.gain[2 * TL + 1 + 2 * CL];
        head.beta = model.bias[2 * TL + 1 + 2 * CL];
        head.y = words + L.c_logits(b, CL);
        put(T.projection_offset(T.head(b)), head);
        Draw d;
        d.book = b;
        d.books = C;
        d.logits = words + L.c_logits(b, CL);
        d.token_words = words + L.c_token(b, CL);
        d.current = a.current;
        d.tokens = a.tokens;
        d.row_base = a.row_base;
        d.step_stride = a.step_stride;
        d.known = a.known;
        d.distributions = a.distributions;
        d.splits = a.splits;
        d.payload = a.payload;
        d.payload_bytes = a.payload_bytes;
        put(T.draw_offset(b), d);
    }
    return table;
}

bool frame_supported(int width, int heads, int head_width, int ffn, int latent, int alphabet, int lanes)
{
    const bool reference = width == 512 && head_width == 128 && ffn == 2048 && latent == 1024;
    const bool wide = width == 1024 && head_width == 64 && ffn == 4096 && latent == 1024;
    return (reference || wide) && heads * head_width == width && alphabet == 1024 && lanes >= 1 &&
           lanes <= max_lanes;
}

std::size_t frame_exchange_words(int width, int ffn, int latent, int alphabet, int books, int temporal_layers,
                                 int codebook_layers)
{
    return Words(width, ffn, latent, alphabet, books, temporal_layers, codebook_layers).total;
}

FrameLaunch frame_step(const FrameArgs& a, hipStream_t stream)
{
    require(frame_supported(a.width, a.heads, a.head_width, a.ffn, a.latent, a.alphabet, a.lanes),
            "frame step: unsupported geometry");
    require(a.steps >= 1 && a.position >= 0 && a.position + a.steps <= a.extent && a.extent <= max_blocks * 64,
            "frame step: position");
    require(a.books >= 1 && a.books <= max_books && a.temporal_layers >= 1 && a.codebook_layers >= 1,
            "frame step: layers");
    require(a.words && a.abort && a.error && a.current && a.tokens && a.row_base && a.jobs && a.epoch != 0,
            "frame step: arguments");
    require(a.known || (a.state && a.payload), "frame step: needs known tokens or a decoder");
    if (a.width == 512)
    {
        return launch_frame<8, 32, 16, 128>(a, stream);
    }
    return launch_frame<16, 64, 16, 64>(a, stream);
}
} // namespace tsac_hip
