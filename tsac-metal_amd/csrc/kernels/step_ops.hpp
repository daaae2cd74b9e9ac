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

// The 24 payload bytes from `from` on, as RangeDecoder::read returns them (zero
// past the end), big-endian in three wave-uniform 64-bit words (byte 0 in the
// top bits of part[0]), and how many of them exist. A symbol's ten decisions
// read at most 20: a decision leaves range >= 1, so at most two renormalising
// shifts follow it.
struct PayloadBytes
{
    uint64_t part[3];
    uint32_t available;
};

// `staged` is 4-byte aligned and holds zeros past the payload's end.
__device__ __forceinline__ PayloadBytes payload_bytes(const ByteWindow& window, unsigned long long from)
{
    PayloadBytes b{{0, 0, 0}, 0};
    const unsigned long long end = uniform64(window.payload_bytes), base = uniform64(window.base);
    const uint32_t size = __builtin_amdgcn_readfirstlane(uint32_t(window.size));
    b.available = from < end ? uint32_t(end - from < 24 ? end - from : 24) : 0u;
    const unsigned long long at = from - base;
    uint32_t word[6] = {0, 0, 0, 0, 0, 0}; // bytes 4i .. 4i + 3, the first on top
    if (at + 28 <= size)
    {
        // Seven aligned words around the 24 bytes, realigned and byte-swapped.
        const Shared<uint32_t> words = (Shared<uint32_t>)(shared(window.staged));
        const uint32_t first = uint32_t(at) / 4, shift = uint32_t(at) % 4;
        uint32_t w[7];
#pragma unroll
        for (int i = 0; i < 7; ++i)
        {
            w[i] = words[first + i];
        }
#pragma unroll
        for (int i = 0; i < 6; ++i)
        {
            const uint32_t little = __builtin_amdgcn_alignbyte(w[i + 1], w[i], shift);
            word[i] = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_perm(little, little, 0x00010203u));
        }
    }
    else
    {
        const Shared<uint8_t> staged = shared(window.staged);
#pragma unroll
        for (uint32_t i = 0; i < 24; ++i)
        {
            uint32_t v = 0;
            if (i < b.available)
            {
                v = at + i < size ? uint32_t(staged[at + i])
                                  : uint32_t(*(const __attribute__((address_space(1))) uint8_t*)(window.payload + from + i));
            }
            word[i / 4] |= __builtin_amdgcn_readfirstlane(v) << (8 * (3 - i % 4));
        }
    }
#pragma unroll
    for (int i = 0; i < 3; ++i)
    {
        b.part[i] = (uint64_t(word[2 * i]) << 32) | word[2 * i + 1];
    }
    return b;
}

// Bytes k .. k + 7 (k <= 16) as a 64-bit queue, byte k on top.
__device__ __forceinline__ uint64_t byte_queue(const PayloadBytes& b, uint32_t k)
{
    const bool low = k < 8;
    const uint64_t first = low ? b.part[0] : b.part[1], second = low ? b.part[1] : b.part[2];
    const uint32_t s = 8 * (k & 7);
    return (first << s) | ((second >> 1) >> (63 - s));
}

// One RangeDecoder::get (src/format/range.cpp:136-152) on wave-uniform values:
// the split, the bit, the interval and the renormalising shifts (one below
// 0xff01, a second below 0x100), with the next payload bytes taken from the
// top of `queue`; node becomes the child taken. Valid states have
// code < range < 2^24, so the comparisons are sign bits of differences (no
// condition register is kept across instructions).
__device__ __forceinline__ void decide(uint32_t& range, uint32_t& code, uint64_t& queue, uint32_t& shifts, int& node,
                                       uint32_t q)
{
    const uint32_t range0 = uint32_t((uint64_t(range) * q) >> 15);
    const int32_t left = int32_t(code - range0) >> 31; // -1 when code < range0: the zero branch
    code -= range0 & ~uint32_t(left);
    range = left ? range0 : range - range0;
    const uint32_t n = (uint32_t(int32_t(range - 0xff01u)) >> 31) + (uint32_t(int32_t(range - 0x100u)) >> 31);
    const uint32_t by = 8 * n;
    range <<= by;
    code = (code << by) | uint32_t((queue >> (63 - by)) >> 1);
    queue <<= by;
    shifts += n;
    // Kept apart so that the child index stays a scalar add (a funnel shift
    // would move it to a vector register and back before the next read).
    int twice = 2 * node;
    __asm__ volatile("" : "+s"(twice));
    node = twice + 1 + left;
}

// One decode_categorical symbol with RangeDecoder::get. Called by a whole wave
// with identical arguments. The ten decisions run one after the other on
// wave-uniform values; each decision's q is read from the lane that holds it
// (v_readlane), so no decision waits for memory: lane l holds q(l) from `top`
// for levels 0..5, and once the node at depth 6 is known, lanes 1..15 compute
// the q's of its subtree for levels 6..9.
//
// RangeDecoder::get fails when a decision leaves code >= range. A decision
// from a state with code < range keeps code < range (the zero branch sets
// range = range0 > code, the one branch subtracts range0 from both, and a
// renormalising shift appends a byte below 256), so a decode fails only from
// a state entered with code >= range, and then at its first decision, which
// goes to the one branch; the symbol and state are those there, as the
// reference leaves them.
__device__ __forceinline__ int decode_symbol(const uint16_t* top, const Masses& mass, DecoderState& s,
                                             const ByteWindow& window)
{
    const int lane = __lane_id();
    if (__builtin_amdgcn_readfirstlane(s.failed))
    {
        return 0;
    }
    const unsigned long long offset = uniform64(s.offset);
    uint32_t range = uint32_t(__builtin_amdgcn_readfirstlane(s.range));
    uint32_t code = uint32_t(__builtin_amdgcn_readfirstlane(s.code));
    const int q_top = int(shared(top)[lane]); // lane 0's entry is not used
    // Lane l: the left masses along the path to node 64 + l.
    float left6[6];
#pragma unroll
    for (int d = 0; d < 6; ++d)
    {
        left6[d] = mass.nodes[2 * ((64 + lane) >> (6 - d))];
    }
    const PayloadBytes bytes = payload_bytes(window, offset);
    uint64_t queue = bytes.part[0];
    uint32_t shifts = 0;
    int node = 1;
    if (code >= range)
    {
        decide(range, code, queue, shifts, node, uint32_t(__builtin_amdgcn_readlane(q_top, 1)));
        s.range = range;
        s.code = code;
        s.offset = offset + min(shifts, bytes.available);
        s.failed = 1;
        return (node << 9) - 1024;
    }
    // Levels 0..5; three decisions read at most six bytes of a queue.
#pragma unroll
    for (int d = 0; d < 6; ++d)
    {
        if (d == 3)
        {
            queue = byte_queue(bytes, shifts);
        }
        decide(range, code, queue, shifts, node, uint32_t(__builtin_amdgcn_readlane(q_top, node)));
    }
    // The mass the walk enters node (64 + lane) with, then node's.
    float entering_lane = 1.0f;
#pragma unroll
    for (int d = 0; d < 6; ++d)
    {
        const bool right = (lane >> (5 - d)) & 1;
        entering_lane = right ? flush(entering_lane - left6[d]) : left6[d];
    }
    const float entering = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(entering_lane), node - 64));
    // Lane u (1..15): q of subtree node u in heap order, node_q15 with every
    // mass read made unconditionally (a leaf only for the own left child at
    // depth 3), so that they go out together.
    int q_sub;
    {
        const int u = (lane & 15) ? (lane & 15) : 1;
        const int depth = 31 - __builtin_clz(uint32_t(u));
        const int n = (node << depth) + (u - (1 << depth));
        float left[3];
#pragma unroll
        for (int d = 0; d < 3; ++d)
        {
            left[d] = mass.nodes[2 * (n >> max(depth - d, 0))];
        }
        const int own = 2 * n; // 256 .. 2047
        const float own_node = mass.nodes[own & 1023];
        const float own_leaf = flush(bf16_to_float(mass.leaves[own & 1023]));
        float e = entering;
#pragma unroll
        for (int d = 0; d < 3; ++d)
        {
            if (d < depth)
            {
                const bool right = (n >> (depth - 1 - d)) & 1;
                e = right ? flush(e - left[d]) : left[d];
            }
        }
        q_sub = q15(own < 1024 ? own_node : own_leaf, e);
    }
    // Levels 6..9; two decisions per queue.
    const int node6 = node;
    node = 1;
#pragma unroll
    for (int d = 0; d < 4; ++d)
    {
        if (d % 2 == 0)
        {
            queue = byte_queue(bytes, shifts);
        }
        decide(range, code, queue, shifts, node, uint32_t(__builtin_amdgcn_readlane(q_sub, node)));
    }
    s.range = range;
    s.code = code;
    s.offset = offset + min(shifts, bytes.available);
    return 16 * node6 + (node - 16) - 1024;
}
} // namespace step
} // namespace tsac_hip
