// Device helpers shared by the decode-side kernels: row-tile addressing, the
// rotary pair rotation, conditional_q15 and the categorical subtree masses.
#pragma once

#include "decode.hpp"
#include "device_numeric.hpp"
#include "row_ops.hpp"

#include <cstddef>

namespace tsac_hip
{
namespace step
{
constexpr int tile_rows = 64;
constexpr int segments = 16;
constexpr int max_columns = 8;

__device__ __forceinline__ std::size_t tile_offset(int t, int b, int s, int blocks)
{
    return ((std::size_t(t) * blocks + b) * segments + s) * (tile_rows * 16);
}

__device__ __forceinline__ void rotate(float& re, float& im, const uint16_t* c)
{
    const float cosine = bf16_to_float(c[0]), sine = bf16_to_float(c[1]);
    const float im_sine = im * sine;
    const float re_sine = re * sine;
    const float r = __builtin_fmaf(re, cosine, -im_sine);
    const float i = __builtin_fmaf(im, cosine, re_sine);
    re = bf16_to_float(float_to_bf16(r));
    im = bf16_to_float(float_to_bf16(i));
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

// Heap-ordered subtree masses of one 1024-symbol row held 16 per lane, into
// nodes[1..1023] (shared memory): node n covers 1024 >> floor(log2 n) symbols
// and has children 2n and 2n + 1. Each mass is the reference's pair tree over
// its leaves (probability_sum, src/format/categorical.cpp:17-30). Whole wave;
// the wave's own later reads of nodes written by other lanes must first wait
// for these writes (lgkmcnt). Returns whether every leaf is finite and
// non-negative.
__device__ __forceinline__ bool build_masses(const float (&leaf)[16], int lane, float* nodes)
{
    bool valid = true;
    float level[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
    {
        valid = valid && is_finite(leaf[2 * i]) && leaf[2 * i] >= 0.0f && is_finite(leaf[2 * i + 1]) &&
                leaf[2 * i + 1] >= 0.0f;
        level[i] = flushed_add(flush(leaf[2 * i]), flush(leaf[2 * i + 1]));
        nodes[512 + lane * 8 + i] = level[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        level[i] = flushed_add(level[2 * i], level[2 * i + 1]);
        nodes[256 + lane * 4 + i] = level[i];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
    {
        level[i] = flushed_add(level[2 * i], level[2 * i + 1]);
        nodes[128 + lane * 2 + i] = level[i];
    }
    float v = flushed_add(level[0], level[1]);
    nodes[64 + lane] = v;
    // Level l spans 32 << l leaves (2 << l lanes); one lane per node stores it.
    const auto store = [&](int l) {
        const int size = 32 << l;
        if ((lane * 16) % size == 0)
        {
            nodes[1024 / size + lane * 16 / size] = v;
        }
    };
    v = butterfly_ftz_add<1>(v);
    store(0);
    v = butterfly_ftz_add<2>(v);
    store(1);
    v = butterfly_ftz_add<4>(v);
    store(2);
    v = butterfly_ftz_add<8>(v);
    store(3);
    v = butterfly_ftz_add<16>(v);
    store(4);
    v = butterfly_ftz_add<32>(v);
    store(5);
    return __all(valid);
}

// Explicit shared-memory views: a generic pointer whose address space the
// compiler cannot see turns shared-memory reads into flat loads.
template <class T> using Shared = const __attribute__((address_space(3))) T*;
template <class T> __device__ __forceinline__ Shared<T> shared(const T* p)
{
    return (Shared<T>)(p);
}

// Decision probabilities of decode_categorical (src/format/categorical.cpp:119-142)
// by bisection-tree node: a walk at node n splits its symbols between children
// 2n and 2n + 1 (nodes 1024..2047 are the symbols) with
// q(n) = conditional_q15(mass(2n), entering(n)). The mass a walk enters with
// depends only on the node: 1 at the root, mass(c) for a left child c, and
// flush(entering(parent) - mass(c - 1)) for a right child c. So q(n) needs no
// walk, only the masses along n's path from an ancestor and the mass the walk
// enters that ancestor with. mass(c) for c >= 1024 is the flushed leaf.
struct Masses
{
    Shared<float> nodes;     // build_masses' nodes[1..1023]
    Shared<uint16_t> leaves; // the row's BF16 probabilities

    __device__ __forceinline__ Masses(const float* n, const uint16_t* l) : nodes(shared(n)), leaves(shared(l))
    {
    }
    __device__ __forceinline__ float operator()(int c) const
    {
        return c < 1024 ? nodes[c] : flush(bf16_to_float(leaves[c - 1024]));
    }
};

// q(node) for `node` `depth` (<= max_depth) levels below its ancestor
// node >> depth, entered with `entering`.
template <int max_depth>
__device__ __forceinline__ uint16_t node_q15(const Masses& mass, float entering, int node, int depth)
{
    float left[max_depth];
#pragma unroll
    for (int d = 0; d < max_depth; ++d)
    {
        left[d] = d < depth ? mass(2 * (node >> (depth - d))) : 0.0f;
    }
    const float own_left = mass(2 * node);
#pragma unroll
    for (int d = 0; d < max_depth; ++d)
    {
        if (d < depth)
        {
            const bool right = (node >> (depth - 1 - d)) & 1;
            entering = right ? flush(entering - left[d]) : left[d];
        }
    }
    return q15(own_left, entering);
}

// encode_categorical (src/format/categorical.cpp:95-117) for a known symbol:
// the Q15 split of each of the ten decisions along its bisection path. Lane k
// (k < 10) returns decision k's: the node at depth k on the path to leaf
// 1024 + symbol, entered from the root with mass 1.
__device__ __forceinline__ uint16_t path_split(const Masses& mass, int symbol, int lane)
{
    const int depth = lane < 10 ? lane : 9;
    return node_q15<9>(mass, 1.0f, (1024 + symbol) >> (10 - depth), depth);
}

// q(1..63), lane l computing node l; lane 0 writes nothing.
__device__ __forceinline__ void build_top_decisions(int lane, const Masses& mass, uint16_t* top)
{
    if (lane != 0)
    {
        top[lane] = node_q15<5>(mass, 1.0f, lane, 31 - __builtin_clz(uint32_t(lane)));
    }
}

// Payload bytes of one launch's decoding staged in shared memory: the window
// after the offset the launch starts at.
struct ByteWindow
{
    const uint8_t* staged; // `size` bytes from `base` on (shared memory)
    int size;
    unsigned long long base;
    const uint8_t* payload; // the whole payload, for reads past the window
    unsigned long long payload_bytes;
};

__device__ __forceinline__ unsigned long long uniform64(unsigned long long v)
{
    return (uint64_t(__builtin_amdgcn_readfirstlane(uint32_t(v >> 32))) << 32) |
           __builtin_amdgcn_readfirstlane(uint32_t(v));
}

// The 16 payload bytes from `from` on, as RangeDecoder::read returns them (zero
// past the end), in four words; and how many of them exist. One replay of at
// most eight decisions reads at most 16: a decision leaves range >= 1, so at
// most two renormalising shifts follow it.
struct Bytes16
{
    uint32_t word[4];
    uint32_t available;

    // Byte k (< 16) by shifts of two 64-bit halves: an index into `word` with a
    // per-lane k would put the array in scratch memory.
    __device__ __forceinline__ uint32_t operator[](uint32_t k) const
    {
        const uint64_t low = word[0] | (uint64_t(word[1]) << 32), high = word[2] | (uint64_t(word[3]) << 32);
        return uint32_t((k < 8 ? low >> (8 * k) : high >> (8 * (k - 8))) & 0xffu);
    }
};

// `staged` is 4-byte aligned and holds zeros past the payload's end.
__device__ __forceinline__ Bytes16 next_bytes(const ByteWindow& window, unsigned long long from)
{
    Bytes16 b{{0, 0, 0, 0}, 0};
    const unsigned long long end = uniform64(window.payload_bytes), base = uniform64(window.base);
    const uint32_t size = __builtin_amdgcn_readfirstlane(uint32_t(window.size));
    b.available = from < end ? uint32_t(end - from < 16 ? end - from : 16) : 0u;
    const unsigned long long at = from - base;
    if (at + 20 <= size)
    {
        // Five aligned words around the 16 bytes, realigned.
        const Shared<uint32_t> words = (Shared<uint32_t>)(shared(window.staged));
        const uint32_t first = uint32_t(at) / 4, shift = uint32_t(at) % 4;
        uint32_t w[5];
#pragma unroll
        for (int i = 0; i < 5; ++i)
        {
            w[i] = words[first + i];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            b.word[i] = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_alignbyte(w[i + 1], w[i], shift));
        }
        return b;
    }
    const Shared<uint8_t> staged = shared(window.staged);
#pragma unroll
    for (uint32_t i = 0; i < 16; ++i)
    {
        uint32_t v = 0;
        if (i < b.available)
        {
            v = at + i < size ? uint32_t(staged[at + i])
                              : uint32_t(*(const __attribute__((address_space(1))) uint8_t*)(window.payload + from + i));
        }
        b.word[i / 4] |= __builtin_amdgcn_readfirstlane(v) << (8 * (i % 4));
    }
    return b;
}

struct Coder
{
    uint32_t range, code;
    uint32_t used; // payload bytes read since the replay's start
};

// RangeDecoder::get (src/format/range.cpp:136-152) forced along a path: for
// decision d the path takes bit (path >> (levels - 1 - d)) & 1 with
// probability-of-zero q[d]. Returns whether every decision the decoder makes
// agrees with the path, up to the end or up to a failure, whose decision
// index goes to `failed_at` (else -1); the state stops there. Branch free.
template <int levels>
__device__ __forceinline__ bool follow(Coder& c, const uint32_t (&q)[levels], int path, int& failed_at,
                                       const Bytes16& bytes)
{
    bool agrees = true, live = true;
    failed_at = -1;
#pragma unroll
    for (int d = 0; d < levels; ++d)
    {
        const bool right = (path >> (levels - 1 - d)) & 1;
        const uint32_t range0 = uint32_t((uint64_t(c.range) * q[d]) >> 15);
        agrees = agrees && (!live || (c.code >= range0) == right);
        uint32_t code = right ? c.code - range0 : c.code;
        uint32_t range = right ? c.range - range0 : range0;
        uint32_t used = c.used;
#pragma unroll
        for (int r = 0; r < 2; ++r)
        {
            const bool shift = range < 0xff01u;
            const bool read = shift && used < bytes.available;
            const uint32_t next = read ? bytes[used] : 0u;
            range = shift ? range << 8 : range;
            code = shift ? (code << 8) + next : code;
            used += read ? 1u : 0u;
        }
        if (live)
        {
            c.code = code;
            c.range = range;
            c.used = used;
        }
        if (live && !(code < range))
        {
            failed_at = d;
            live = false;
        }
    }
    return agrees;
}

__device__ __forceinline__ Coder kept_coder(const Coder& c, int lane)
{
    return Coder{uint32_t(__builtin_amdgcn_readlane(int(c.range), lane)),
                 uint32_t(__builtin_amdgcn_readlane(int(c.code), lane)),
                 uint32_t(__builtin_amdgcn_readlane(int(c.used), lane))};
}

// One decode_categorical symbol with RangeDecoder::get. Called by a whole wave
// with identical arguments. Instead of making the ten decisions one after the
// other, lane j replays the first six along path j (the decisions' q from
// `top`) and the lane whose path the decoder agrees with is kept; then 16
// lanes do the same for the last four, below the node reached, with q
// computed on the spot. Each replay is the reference's arithmetic, so the
// kept lane's state is the serial decoder's. On a failure the symbol and
// state are those at the failing decision, as the reference leaves them.
__device__ __forceinline__ int decode_symbol(const uint16_t* top, const Masses& mass, DecoderState& s,
                                             const ByteWindow& window)
{
    const int lane = __lane_id();
    if (__builtin_amdgcn_readfirstlane(s.failed))
    {
        return 0;
    }
    const unsigned long long offset = uniform64(s.offset);
    const Coder start{uint32_t(__builtin_amdgcn_readfirstlane(s.range)),
                      uint32_t(__builtin_amdgcn_readfirstlane(s.code)), 0u};
    const Shared<uint16_t> shared_top = shared(top);
    // Levels 0..5: path = lane.
    uint32_t q6[6];
    float left6[6];
#pragma unroll
    for (int d = 0; d < 6; ++d)
    {
        const int node = (64 + lane) >> (6 - d);
        q6[d] = shared_top[node];
        left6[d] = mass.nodes[2 * node];
    }
    const Bytes16 bytes6 = next_bytes(window, offset);
    Coder c = start;
    int failed_at;
    const bool agrees = follow<6>(c, q6, lane, failed_at, bytes6);
    const int j = __builtin_ctzll(__ballot(agrees)); // some lane always agrees
    const int fail6 = __builtin_amdgcn_readlane(failed_at, j);
    const Coder at = kept_coder(c, j);
    const unsigned long long offset6 = offset + at.used;
    if (fail6 >= 0)
    {
        s.range = at.range;
        s.code = at.code;
        s.offset = offset6;
        s.failed = 1;
        const int node = (1 << (fail6 + 1)) + (j >> (5 - fail6)); // after fail6 + 1 decisions
        return (node << (9 - fail6)) - 1024;
    }
    // Mass entering node 64 + j.
    float entering = 1.0f;
#pragma unroll
    for (int d = 0; d < 6; ++d)
    {
        const bool right = (lane >> (5 - d)) & 1;
        entering = right ? flush(entering - left6[d]) : left6[d];
    }
    const int node6 = 64 + j;
    entering = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(entering), j));
    // Levels 6..9: lane u in 1..15 computes q of node6's subtree node u (heap
    // order: node (node6 << depth) + u - (1 << depth)), then lanes 0..15
    // replay path = lane, whose d-th node is subtree node (16 + lane) >> (4 - d).
    const Bytes16 bytes4 = next_bytes(window, offset6);
    uint32_t mine = 0;
    if (lane >= 1 && lane < 16)
    {
        const int depth = 31 - __builtin_clz(uint32_t(lane));
        mine = node_q15<3>(mass, entering, (node6 << depth) + (lane - (1 << depth)), depth);
    }
    uint32_t q4[4];
#pragma unroll
    for (int d = 0; d < 4; ++d)
    {
        q4[d] = uint32_t(__shfl(int(mine), (16 + (lane & 15)) >> (4 - d), wave));
    }
    Coder c2{at.range, at.code, 0u};
    int failed2;
    const bool agrees2 = follow<4>(c2, q4, lane & 15, failed2, bytes4) && lane < 16;
    const int j2 = __builtin_ctzll(__ballot(agrees2));
    const int fail4 = __builtin_amdgcn_readlane(failed2, j2);
    const Coder end = kept_coder(c2, j2);
    s.range = end.range;
    s.code = end.code;
    s.offset = offset6 + end.used;
    if (fail4 >= 0)
    {
        s.failed = 1;
        const int node = (node6 << (fail4 + 1)) + (j2 >> (3 - fail4)); // after 7 + fail4 decisions
        return (node << (3 - fail4)) - 1024;
    }
    return 16 * node6 + j2 - 1024;
}

} // namespace step
} // namespace tsac_hip
