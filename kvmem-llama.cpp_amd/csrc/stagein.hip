// Stage-in: F16 KV rows -> ggml q8_0 / q5_0 / q4_0 (or F16) rows scattered
// into pool slots.  HBM-bound: every F16 byte is read once with 16-byte
// coalesced loads and every output byte is written once with 16-byte stores.
//
// Work decomposition.  An operation (one block of one layer of K or V) is a
// linear run of 32-element groups (rows are contiguous groups and the
// output rows of a slot are contiguous cells).  A workgroup of 256 threads
// handles a chunk of 512 groups, eight 16-group rounds per wave with all
// eight 16-byte loads of a lane in flight together; inside a wave, four
// consecutive lanes own one group (8 halves = 16 bytes each), so a
// wave-wide load instruction reads 1 KiB of contiguous F16.  Output goes
// out with nontemporal 16-byte stores.  The group scale comes from a two-step
// quad reduction through DPP, the quantized bytes are packed in registers,
// written to the wave's LDS region in ggml's byte layout, and copied out
// with aligned 16-byte global stores (2-byte stores into a slot that is not
// a whole number of 16 bytes, which starts 2-byte aligned only).
//
// Arithmetic follows ggml's quantize_row_*_ref exactly (restated in the
// reference's CUDA kernels, llama-kvmem-stagein.cu:180-233):
//   q8_0: d = amax/127, id = d ? 1/d : 0, q = roundf(x*id) (|x*id| <= 127)
//   q4_0: d = vmax/-8,  q = min(15, trunc(x*id + 8.5))
//   q5_0: d = vmax/-16, q = min(31, trunc(x*id + 16.5)), bit 4 -> qh
// (division by -8 / -16 is done as the exactly equal multiplication by
// -0.125 / -0.0625: both round the same exact quotient once)
// where vmax is the first element of largest magnitude.  The products and
// sums are separate IEEE operations (no FMA contraction in this file),
// the divisions are correctly rounded (computed by the exact shortcuts
// scale_div127 / scale_recip below), d is stored as f16 RNE.
//
// With a pool transform the rows are widened to fp32, RoPE'd (K) and
// Hadamard-rotated before they are quantized, as the reference's raw-K
// stage-in does (llama-kvmem-stagein.cu:704-740).  A head never straddles a
// 16-group round (head_dim divides 512), so a rotary pair and a butterfly
// partner are always lanes of the same wave: RoPE pairs are exchanged with
// one lane shuffle, butterfly spans 1, 2, 4 stay inside a lane and spans
// 8 .. width/2 exchange with lane ^ span/8.  The cos/sin of every (row,
// rotary pair) of a chunk are computed once per workgroup into LDS.
#include "kvmem_internal.hpp"
#include "device_reselect.h"
#include "move_plan.hpp"

#include <algorithm>
#include <cstring>
#include <vector>

#pragma clang fp contract(off)

namespace kvmem_hip {

// A workgroup of 4 waves takes a chunk of 4 * 16 * R groups: each wave R
// rounds of 16 groups, all R 16-byte loads of a lane in flight.  R by
// output format, as measured on 77-block jobs at random block ids and slots
// (fraction of HBM peak at R = 4 / 8 / 16): q8_0 0.70 / 0.66 / 0.66,
// q5_0 0.64 / 0.67 / 0.67, q4_0 0.67 / 0.68 / 0.67, F16 0.71 / 0.70 / 0.72.
// With the row transform (VALU-bound) every format uses 8, which bounds the
// rows of a chunk's RoPE table.
__host__ __device__ constexpr int rounds_of(int type, bool xf) {
    return xf ? 8 : type == KVMEM_TYPE_Q8_0 ? 4 : type == KVMEM_TYPE_F16 ? 16 : 8;
}
__host__ __device__ constexpr uint32_t chunk_groups_of(int type, bool xf) {
    return 64u * static_cast<uint32_t>(rounds_of(type, xf));
}
constexpr int kTabMax = 4096;  // (row, rotary pair) entries per chunk
// Layers of one block a workgroup takes when K is RoPE'd (one table build).
constexpr uint32_t kRopeLayerGroup = 4;

// Rows of `gpr` groups that one chunk of `cg` groups can touch.
inline uint32_t chunk_rows_of(uint32_t gpr, uint32_t cg) {
    return (cg % gpr == 0) ? cg / gpr : (cg - 1) / gpr + 2;
}

template <int TYPE> struct Fmt;
template <> struct Fmt<KVMEM_TYPE_Q8_0> { static constexpr int GB = 34; };
template <> struct Fmt<KVMEM_TYPE_Q4_0> { static constexpr int GB = 18; };
template <> struct Fmt<KVMEM_TYPE_Q5_0> { static constexpr int GB = 22; };
template <> struct Fmt<KVMEM_TYPE_F16> { static constexpr int GB = 64; };

// A contiguous run of groups of one operation.
struct Chunk {
    const uint8_t *src;   // first byte of the operation's F16 rows
    uint8_t *dst;         // first byte of the operation's output rows
    uint32_t g0;          // first group of this chunk within the operation
    uint32_t ng;          // groups in this chunk (<= the source's chunk_groups)
    uint32_t gpr;         // groups per row
    uint32_t src_stride;  // bytes between F16 rows
    int32_t pos0;         // position of the operation's row 0 (RoPE)
};

// Source 1: an explicit list of operations.  chunk0 is the index of the
// operation's first chunk; the list is sorted by it.
struct QuantOpDev {
    const uint8_t *src;
    uint8_t *dst;
    uint32_t n_groups;
    uint32_t gpr;
    uint32_t src_stride;
    uint32_t chunk0;
};

struct OpListSource {
    const QuantOpDev *ops;
    uint32_t n_ops;
    uint32_t chunk_groups;  // chunk_groups_of(type, false)
    __device__ bool chunk(uint32_t c, Chunk &out) const {
        uint32_t lo = 0, hi = n_ops;  // last op with chunk0 <= c
        while (hi - lo > 1) {
            const uint32_t mid = (lo + hi) >> 1;
            if (ops[mid].chunk0 <= c) {
                lo = mid;
            } else {
                hi = mid;
            }
        }
        const QuantOpDev op = ops[lo];
        out.src = op.src;
        out.dst = op.dst;
        out.g0 = (c - op.chunk0) * chunk_groups;
        if (out.g0 >= op.n_groups) {
            return false;
        }
        out.ng = min(chunk_groups, op.n_groups - out.g0);
        out.gpr = op.gpr;
        out.src_stride = op.src_stride;
        out.pos0 = 0;
        return true;
    }
    __device__ void bind(const ArgTables &) {}  // the op list is always uploaded
    // rows may be strided; no row transform on this source
    static constexpr bool kContiguous = false;
    static constexpr uint32_t head_dim = 32, n_rot = 0, hadamard = 0;
    static constexpr float hscale = 1.0f;
    static constexpr const float *theta = nullptr;
};

// Source 2: whole blocks of a history, for every layer.  Item i names a
// source block (addressing index), its destination slot, its tokens and
// the position of its token 0.
//   src(item, layer) = base + block*block_stride + layer*layer_stride
//   dst(item, layer) = layer_dst[layer] + slot*block_tokens*row_bytes
struct BlockSource {
    static constexpr bool kContiguous = true;  // group g of an operation at src + 64 g
    const uint8_t *base;
    // set by bind() from the job's tables:
    const uint8_t *const *layer_dst;  // [n_layers]
    const uint32_t *items;            // [n_items][4]: block, slot, n_tokens, pos0
    const float *theta;               // [n_rot/2] (RoPE)
    const uint8_t *tables;            // the job's uploaded tables, or null: in the kernel's ArgTables
    uint32_t layer_off, items_off, theta_off;  // byte offsets of the three tables in them
    uint64_t block_stride;
    uint64_t layer_stride;
    uint32_t n_layers;
    uint32_t block_tokens;
    uint32_t gpr;
    uint32_t row_bytes;               // output bytes per row
    uint32_t chunk_groups;            // chunk_groups_of(type, transform on)
    uint32_t chunks_per_op;           // ceil(block_tokens*gpr / chunk_groups)
    uint32_t head_dim;                // transform: head width (power of two)
    uint32_t n_rot;                   // RoPE rotary dims (0 = none)
    uint32_t hadamard;                // Hadamard width (0 = none)
    float hscale;                     // 1 / sqrtf(hadamard)
    uint32_t layer_group;             // layers per workgroup chunk index (RoPE'd K: 4; else 1)
    __device__ void bind(const ArgTables &t) {
        const uint8_t *b = table_base(tables, t);
        layer_dst = reinterpret_cast<const uint8_t *const *>(b + layer_off);
        items = reinterpret_cast<const uint32_t *>(b + items_off);
        theta = reinterpret_cast<const float *>(b + theta_off);
    }
    __device__ bool chunk(uint32_t c, Chunk &out) const {
        const uint32_t op = c / chunks_per_op;
        const uint32_t sub = c - op * chunks_per_op;
        const uint32_t item = op / n_layers;
        return chunk_at(item, op - item * n_layers, sub, out);
    }
    // Chunk `sub` of the run of (item, layer).  Tables in device memory
    // (uploaded, or written by an earlier kernel) are read through the
    // constant address space: uniform scalar loads, as the argument bytes
    // are, instead of vector loads the chunk's addresses would wait on.
    __device__ bool chunk_at(uint32_t item, uint32_t layer, uint32_t sub, Chunk &out) const {
        uint32_t block, slot, ntok;
        const uint8_t *ldst;
        if (tables) {
            const u32x4_t it = cload<u32x4_t>(tables, items_off + 16u * item);
            block = it[0];
            slot = it[1];
            ntok = it[2];
            out.pos0 = static_cast<int32_t>(it[3]);
            ldst = reinterpret_cast<const uint8_t *>(cload<uint64_t>(tables, layer_off + 8u * layer));
        } else {
            block = items[4 * item + 0];
            slot = items[4 * item + 1];
            ntok = items[4 * item + 2];
            out.pos0 = static_cast<int32_t>(items[4 * item + 3]);
            ldst = layer_dst[layer];
        }
        const uint32_t total = ntok * gpr;
        out.g0 = sub * chunk_groups;
        if (out.g0 >= total) {
            return false;
        }
        out.ng = min(chunk_groups, total - out.g0);
        out.src = base + block * block_stride + layer * layer_stride;
        out.dst = const_cast<uint8_t *>(ldst) + static_cast<uint64_t>(slot) * block_tokens * row_bytes;
        out.gpr = gpr;
        out.src_stride = gpr * 64u;
        return true;
    }
};

// ---------------------------------------------------------------- lanes

// Quad exchange through DPP: lane i of each 4-lane quad reads lane i^1 / i^2.
__device__ inline uint32_t quad_xor1(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0xB1, 0xF, 0xF, true));
}
__device__ inline uint32_t quad_xor2(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x4E, 0xF, 0xF, true));
}

__device__ inline float half_bits_to_float(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

__device__ inline uint32_t float_to_half_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));  // v_cvt_f16_f32, RNE
}

__device__ inline void unpack8(const uint4 &v, uint32_t h[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h[2 * i] = w[i] & 0xffffu;
        h[2 * i + 1] = w[i] >> 16;
    }
}

__device__ inline void store_u16(uint8_t *p, uint32_t v) {
    *reinterpret_cast<uint16_t *>(p) = static_cast<uint16_t>(v);
}

// Eight bytes packed in two words -> four 2-byte LDS stores (the group
// layouts only guarantee 2-byte alignment).
__device__ inline void store_8bytes(uint8_t *p, uint32_t lo, uint32_t hi) {
    store_u16(p + 0, lo & 0xffffu);
    store_u16(p + 2, lo >> 16);
    store_u16(p + 4, hi & 0xffffu);
    store_u16(p + 6, hi >> 16);
}

// The quantizers' scale arithmetic without the IEEE division sequence.
// scale_div127(a) = a / 127 for every non-negative float a: the product with
// the rounded reciprocal of 127 corrected by one exact residual (two FMAs);
// scale_recip(d) = 1 / d for every normal |d| <= 2^126 (q8_0/q4_0/q5_0 scales
// never exceed 2^125): the hardware reciprocal refined by one Newton step.
// Both equal the correctly rounded quotients over their whole ranges (checked
// exhaustively by kvmem_hip_check_scale_arith on the device).
__device__ inline float scale_div127(float a) {
    constexpr float r127 = 1.0f / 127.0f;
    const float q0 = a * r127;
    return __builtin_fmaf(__builtin_fmaf(-q0, 127.0f, a), r127, q0);
}

__device__ inline float scale_recip(float d) {
    const float r0 = __builtin_amdgcn_rcpf(d);
    return __builtin_fmaf(__builtin_fmaf(-d, r0, 1.0f), r0, r0);
}

// roundf (half away from zero) of |s| < 128.5, the range of q8_0's x*id:
// truncation of s + copysign(0.49999997f, s) (the float below 0.5) equals
// roundf for every float in that range (checked exhaustively over all of
// them), in three instructions instead of roundf's compare-and-fix.
__device__ inline int round_q8(float s) {
    return static_cast<int>(s + copysignf(0x1.fffffep-2f, s));
}

// Quantize the 8 elements a lane owns (elements 8q..8q+7 of its group) and
// write its share of the group's bytes to `g` (the group's LDS bytes).
template <int TYPE>
__device__ inline void quant_quarter(const uint4 &v, uint32_t q, uint8_t *g, bool valid);

template <>
__device__ inline void quant_quarter<KVMEM_TYPE_Q8_0>(const uint4 &v, uint32_t q, uint8_t *g,
                                                       bool valid) {
    uint32_t h[8];
    unpack8(v, h);
    float x[8];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        x[i] = half_bits_to_float(h[i]);
        amax = fmaxf(amax, fabsf(x[i]));
    }
    amax = fmaxf(amax, __uint_as_float(quad_xor1(__float_as_uint(amax))));
    amax = fmaxf(amax, __uint_as_float(quad_xor2(__float_as_uint(amax))));
    const float d = scale_div127(amax);
    const float id = d != 0.0f ? scale_recip(d) : 0.0f;
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int c = round_q8(x[i] * id);
        w[i >> 2] |= (static_cast<uint32_t>(c) & 0xffu) << (8 * (i & 3));
    }
    if (valid) {
        if (q == 0) {
            store_u16(g, float_to_half_bits(d));
        }
        store_8bytes(g + 2 + 8 * q, w[0], w[1]);
    }
}

// vmax of ggml's q4_0/q5_0: the FIRST element of largest magnitude (strict
// `amax < |v|` scan).  Reduced as a max over keys
//   |h| << 17 | (31 - e) << 1 | sign(h)
// (larger magnitude wins, then lower element index e).  One funnel shift per
// element rotates an f16 of the lane's packed words into place (its sign to
// bit 0, its magnitude to bits 17..31) and one and-or drops the other half
// and inserts the element's index within the lane; the lane's part of the
// index is added after the lane's own max.  An all-zero group keeps
// ggml's initial vmax = +0.
__device__ inline float quad_vmax(const uint4 &v, uint32_t q) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t key = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        // element 2j sits in the low half, 2j + 1 in the high half
        const uint32_t k0 = (__builtin_amdgcn_alignbit(w[j], w[j], 15) & 0xFFFE0001u) |
                            static_cast<uint32_t>((7 - 2 * j) << 1);
        const uint32_t k1 = (__builtin_amdgcn_alignbit(w[j], w[j], 31) & 0xFFFE0001u) |
                            static_cast<uint32_t>((6 - 2 * j) << 1);
        key = max(key, max(k0, k1));
    }
    key |= (3u - q) << 4;
    uint32_t o = quad_xor1(key);
    key = o > key ? o : key;
    o = quad_xor2(key);
    key = o > key ? o : key;
    const uint32_t mag = key >> 17;
    if (mag == 0) {
        return 0.0f;
    }
    return half_bits_to_float(mag | ((key & 1u) << 15));
}

template <int TOP>
__device__ inline uint32_t trunc_code(float x, float id, float bias) {
    const float s = x * id;     // rounded product
    const float t = s + bias;   // rounded sum (separate operation)
    const int c = static_cast<int>(t);
    return static_cast<uint32_t>(c < TOP ? c : TOP);
}

// Codes of the 8 elements a lane owns, one per byte: element i of the lane
// in byte i % 4 of word i / 4 (codes fit in 5 bits).
template <int TOP>
__device__ inline void trunc_codes(const uint32_t h[8], float id, float bias, uint32_t &w0,
                                   uint32_t &w1) {
    w0 = 0u;
    w1 = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        w0 |= trunc_code<TOP>(half_bits_to_float(h[i]), id, bias) << (8 * i);
        w1 |= trunc_code<TOP>(half_bits_to_float(h[i + 4]), id, bias) << (8 * i);
    }
}

template <>
__device__ inline void quant_quarter<KVMEM_TYPE_Q4_0>(const uint4 &v, uint32_t q, uint8_t *g,
                                                       bool valid) {
    uint32_t h[8];
    unpack8(v, h);
    const float vmax = quad_vmax(v, q);
    const float d = vmax * -0.125f;        // == vmax / -8 (exact scaling)
    const float id = d != 0.0f ? scale_recip(d) : 0.0f;
    uint32_t w0, w1;
    trunc_codes<15>(h, id, 8.5f, w0, w1);
    // qs[j] = code(j) | code(j + 16) << 4: lanes 0 and 1 write the bytes,
    // the partner code j + 16 sits in the same byte of lane q + 2
    const uint32_t p0 = quad_xor2(w0);
    const uint32_t p1 = quad_xor2(w1);
    if (valid) {
        if (q == 0) {
            store_u16(g, float_to_half_bits(d));
        }
        if (q < 2) {
            store_8bytes(g + 2 + 8 * q, w0 | (p0 << 4), w1 | (p1 << 4));
        }
    }
}

// Bit 4 of each of the 4 bytes of w, as a 4-bit value (byte i -> bit i).
__device__ inline uint32_t bit4_of_bytes(uint32_t w) {
    const uint32_t x = (w >> 4) & 0x01010101u;
    return (x * 0x01020408u) >> 24;  // bits 0, 8, 16, 24 -> 24..27, no carries
}

template <>
__device__ inline void quant_quarter<KVMEM_TYPE_Q5_0>(const uint4 &v, uint32_t q, uint8_t *g,
                                                       bool valid) {
    uint32_t h[8];
    unpack8(v, h);
    const float vmax = quad_vmax(v, q);
    const float d = vmax * -0.0625f;       // == vmax / -16 (exact scaling)
    const float id = d != 0.0f ? scale_recip(d) : 0.0f;
    uint32_t w0, w1;
    trunc_codes<31>(h, id, 16.5f, w0, w1);
    // qh bit e = bit 4 of the code of element e (e = 8q + i)
    uint32_t qh = (bit4_of_bytes(w0) | (bit4_of_bytes(w1) << 4)) << (8 * q);
    qh |= quad_xor1(qh);
    qh |= quad_xor2(qh);
    w0 &= 0x0f0f0f0fu;
    w1 &= 0x0f0f0f0fu;
    const uint32_t p0 = quad_xor2(w0);
    const uint32_t p1 = quad_xor2(w1);
    if (valid) {
        if (q == 0) {
            store_u16(g, float_to_half_bits(d));
            store_u16(g + 2, qh & 0xffffu);
            store_u16(g + 4, qh >> 16);
        }
        if (q < 2) {
            store_8bytes(g + 6 + 8 * q, w0 | (p0 << 4), w1 | (p1 << 4));
        }
    }
}

template <>
__device__ inline void quant_quarter<KVMEM_TYPE_F16>(const uint4 &v, uint32_t q, uint8_t *g,
                                                      bool valid) {
    if (valid) {
        *reinterpret_cast<uint4 *>(g + 16 * q) = v;
    }
}

// ------------------------------------------------- transformed (fp32) rows

// sin and cos of an fp32 angle.  The angle is reduced by pi/2 in double
// (Cody-Waite: k = rint(a * 2/pi), r = a - k*pi/2 with pi/2 split into two
// doubles, one fused multiply-add each), the Taylor series of sin (to r^17)
// and cos (to r^16) are summed by Horner's rule on |r| <= pi/4 (truncation
// below 1e-17), and each result is rounded once to fp32.  Every step is one
// correctly rounded IEEE operation, so a C restatement of the same steps
// reproduces the same bits.  Angles are finite with |a| < 2^40 (a RoPE
// angle is an int32 position times a frequency of at most one).
__device__ inline void rope_sincos(float a, float &sn, float &cs) {
    const double x = static_cast<double>(a);
    const double k = __builtin_rint(x * 0x1.45f306dc9c883p-1);
    double r = x;  // |a| < pi/4: no reduction (keeps the sign of zero)
    if (k != 0.0) {
        r = __builtin_fma(-k, 0x1.921fb54442d18p+0, x);
        r = __builtin_fma(-k, 0x1.1a62633145c07p-54, r);
    }
    const double r2 = r * r;
    double ps = 0x1.952c77030ad4ap-49;
    ps = __builtin_fma(ps, r2, -0x1.ae7f3e733b81fp-41);
    ps = __builtin_fma(ps, r2, 0x1.6124613a86d09p-33);
    ps = __builtin_fma(ps, r2, -0x1.ae64567f544e4p-26);
    ps = __builtin_fma(ps, r2, 0x1.71de3a556c734p-19);
    ps = __builtin_fma(ps, r2, -0x1.a01a01a01a01ap-13);
    ps = __builtin_fma(ps, r2, 0x1.1111111111111p-7);
    ps = __builtin_fma(ps, r2, -0x1.5555555555555p-3);
    double pc = 0x1.ae7f3e733b81fp-45;
    pc = __builtin_fma(pc, r2, -0x1.93974a8c07c9dp-37);
    pc = __builtin_fma(pc, r2, 0x1.1eed8eff8d898p-29);
    pc = __builtin_fma(pc, r2, -0x1.27e4fb7789f5cp-22);
    pc = __builtin_fma(pc, r2, 0x1.a01a01a01a01ap-16);
    pc = __builtin_fma(pc, r2, -0x1.6c16c16c16c17p-10);
    pc = __builtin_fma(pc, r2, 0x1.5555555555555p-5);
    pc = __builtin_fma(pc, r2, -0.5);
    const double sr = r == 0.0 ? r : __builtin_fma(r * r2, ps, r);  // sin(+-0) = +-0
    const double cr = __builtin_fma(r2, pc, 1.0);
    const int quadrant = static_cast<int>(k - 4.0 * __builtin_floor(k * 0.25));  // k mod 4, exact
    const double sv = (quadrant & 1) ? cr : sr;
    const double cv = (quadrant & 1) ? sr : cr;
    sn = static_cast<float>((quadrant & 2) ? -sv : sv);
    cs = static_cast<float>(((quadrant + 1) & 2) ? -cv : cv);
}

// The value of lane ^ M: DPP quad permutes for 1 and 2, a row rotation by
// 8 (within 16 lanes, the same as ^ 8), ds_swizzle's xor mode for 4 and 16
// (within 32 lanes; these run on the LDS pipe, off the VALU that bounds the
// transform), a lane permute for 32.  Every lane of the wave must be active.
template <uint32_t M>
__device__ inline float lane_xor(float v) {
    const int x = __float_as_int(v);
    int r;
    if constexpr (M == 1) {
        r = __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, true);
    } else if constexpr (M == 2) {
        r = __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, true);
    } else if constexpr (M == 4) {
        r = __builtin_amdgcn_ds_swizzle(x, 0x1F | (4 << 10));
    } else if constexpr (M == 8) {
        r = __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, true);  // row_ror:8
    } else if constexpr (M == 16) {
        r = __builtin_amdgcn_ds_swizzle(x, 0x1F | (16 << 10));
    } else {
        r = __shfl_xor(x, static_cast<int>(M), 64);
    }
    return __int_as_float(r);
}

// One butterfly stage of span 8*M across lanes: the lane whose bit M is set
// holds the upper element and keeps partner - own, the other own + partner
// (p + (-x) is the IEEE subtraction p - x).
template <uint32_t M>
__device__ inline void butterfly_lanes(float x[8], uint32_t lane) {
    const uint32_t flip = (lane & M) ? 0x80000000u : 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float p = lane_xor<M>(x[i]);
        x[i] = p + __uint_as_float(__float_as_uint(x[i]) ^ flip);
    }
}

// Walsh-Hadamard rotation of runs of `width` elements, in the order of the
// reference's fwht_kernel: scale every element, then butterflies of span
// 1, 2, 4 (inside the lane) and 8 .. width/2 (partner lane ^ span/8).
__device__ inline void fwht_lanes(float x[8], uint32_t width, float scale, uint32_t lane) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        x[i] = x[i] * scale;
    }
#pragma unroll
    for (int h = 1; h < 8; h <<= 1) {
#pragma unroll
        for (int i = 0; i < 8; i += 2 * h) {
#pragma unroll
            for (int j = 0; j < h; ++j) {
                const float a = x[i + j];
                const float b = x[i + j + h];
                x[i + j] = a + b;
                x[i + j + h] = a - b;
            }
        }
    }
    // width is uniform: whole stages are skipped together
    butterfly_lanes<1>(x, lane);
    butterfly_lanes<2>(x, lane);
    butterfly_lanes<4>(x, lane);
    if (width > 64u) {
        butterfly_lanes<8>(x, lane);
    }
    if (width > 128u) {
        butterfly_lanes<16>(x, lane);
    }
    if (width > 256u) {
        butterfly_lanes<32>(x, lane);
    }
}

// Partner values of a RoPE pair: lane ^ (n_rot/16) when that is a power of
// two (a head's first-half lanes then differ from their partners in exactly
// that bit), else lane +- n_rot/16 through a general lane permute.
__device__ inline void rope_partners(const float x[8], float p[8], uint32_t n_rot, uint32_t lane,
                                     bool rot, bool first) {
    const uint32_t d = n_rot / 16u;
#define KVMEM_XOR_CASE(M)                     \
    case M:                                   \
        for (int i = 0; i < 8; ++i) {         \
            p[i] = lane_xor<M>(x[i]);         \
        }                                     \
        return;
    switch (d) {
        KVMEM_XOR_CASE(1)
        KVMEM_XOR_CASE(2)
        KVMEM_XOR_CASE(4)
        KVMEM_XOR_CASE(8)
        KVMEM_XOR_CASE(16)
        KVMEM_XOR_CASE(32)
        default: break;
    }
#undef KVMEM_XOR_CASE
    const int src = static_cast<int>(rot ? (first ? lane + d : lane - d) : lane);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        p[i] = __shfl(x[i], src, 64);
    }
}

// vmax of ggml's q4_0/q5_0 over fp32 values: the first element of largest
// magnitude (NaNs never win, as in the reference's strict `amax < |v|`);
// an all-zero group keeps the initial vmax = +0.
__device__ inline float quad_vmax_f(const float x[8], uint32_t q) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        amax = fmaxf(amax, fabsf(x[i]));
    }
    amax = fmaxf(amax, __uint_as_float(quad_xor1(__float_as_uint(amax))));
    amax = fmaxf(amax, __uint_as_float(quad_xor2(__float_as_uint(amax))));
    uint32_t key = 0xffffffffu;  // (element << 1) | sign of the first maximum
#pragma unroll
    for (int i = 7; i >= 0; --i) {
        if (fabsf(x[i]) == amax) {
            key = ((8u * q + i) << 1) | (__float_as_uint(x[i]) >> 31);
        }
    }
    uint32_t o = quad_xor1(key);
    key = o < key ? o : key;
    o = quad_xor2(key);
    key = o < key ? o : key;
    return amax == 0.0f ? 0.0f : ((key & 1u) ? -amax : amax);
}

template <int TYPE>
__device__ inline void quant_quarter_f(const float x[8], uint32_t q, uint8_t *g, bool valid);

template <>
__device__ inline void quant_quarter_f<KVMEM_TYPE_Q8_0>(const float x[8], uint32_t q, uint8_t *g,
                                                         bool valid) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        amax = fmaxf(amax, fabsf(x[i]));
    }
    amax = fmaxf(amax, __uint_as_float(quad_xor1(__float_as_uint(amax))));
    amax = fmaxf(amax, __uint_as_float(quad_xor2(__float_as_uint(amax))));
    const float d = scale_div127(amax);
    const float id = d != 0.0f ? scale_recip(d) : 0.0f;
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int c = round_q8(x[i] * id);
        w[i >> 2] |= (static_cast<uint32_t>(c) & 0xffu) << (8 * (i & 3));
    }
    if (valid) {
        if (q == 0) {
            store_u16(g, float_to_half_bits(d));
        }
        store_8bytes(g + 2 + 8 * q, w[0], w[1]);
    }
}

template <int TOP>
__device__ inline void trunc_codes_f(const float x[8], float id, float bias, uint32_t &w0,
                                     uint32_t &w1) {
    w0 = 0u;
    w1 = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        w0 |= trunc_code<TOP>(x[i], id, bias) << (8 * i);
        w1 |= trunc_code<TOP>(x[i + 4], id, bias) << (8 * i);
    }
}

template <>
__device__ inline void quant_quarter_f<KVMEM_TYPE_Q4_0>(const float x[8], uint32_t q, uint8_t *g,
                                                         bool valid) {
    const float vmax = quad_vmax_f(x, q);
    const float d = vmax * -0.125f;        // == vmax / -8 (exact scaling)
    const float id = d != 0.0f ? scale_recip(d) : 0.0f;
    uint32_t w0, w1;
    trunc_codes_f<15>(x, id, 8.5f, w0, w1);
    const uint32_t p0 = quad_xor2(w0);
    const uint32_t p1 = quad_xor2(w1);
    if (valid) {
        if (q == 0) {
            store_u16(g, float_to_half_bits(d));
        }
        if (q < 2) {
            store_8bytes(g + 2 + 8 * q, w0 | (p0 << 4), w1 | (p1 << 4));
        }
    }
}

template <>
__device__ inline void quant_quarter_f<KVMEM_TYPE_Q5_0>(const float x[8], uint32_t q, uint8_t *g,
                                                         bool valid) {
    const float vmax = quad_vmax_f(x, q);
    const float d = vmax * -0.0625f;       // == vmax / -16 (exact scaling)
    const float id = d != 0.0f ? scale_recip(d) : 0.0f;
    uint32_t w0, w1;
    trunc_codes_f<31>(x, id, 16.5f, w0, w1);
    uint32_t qh = (bit4_of_bytes(w0) | (bit4_of_bytes(w1) << 4)) << (8 * q);
    qh |= quad_xor1(qh);
    qh |= quad_xor2(qh);
    w0 &= 0x0f0f0f0fu;
    w1 &= 0x0f0f0f0fu;
    const uint32_t p0 = quad_xor2(w0);
    const uint32_t p1 = quad_xor2(w1);
    if (valid) {
        if (q == 0) {
            store_u16(g, float_to_half_bits(d));
            store_u16(g + 2, qh & 0xffffu);
            store_u16(g + 4, qh >> 16);
        }
        if (q < 2) {
            store_8bytes(g + 6 + 8 * q, w0 | (p0 << 4), w1 | (p1 << 4));
        }
    }
}

template <>
__device__ inline void quant_quarter_f<KVMEM_TYPE_F16>(const float x[8], uint32_t q, uint8_t *g,
                                                        bool valid) {
    if (valid) {
        uint4 v;
        v.x = float_to_half_bits(x[0]) | (float_to_half_bits(x[1]) << 16);
        v.y = float_to_half_bits(x[2]) | (float_to_half_bits(x[3]) << 16);
        v.z = float_to_half_bits(x[4]) | (float_to_half_bits(x[5]) << 16);
        v.w = float_to_half_bits(x[6]) | (float_to_half_bits(x[7]) << 16);
        *reinterpret_cast<uint4 *>(g + 16 * q) = v;
    }
}

// The transformed rounds of a chunk: cos/sin table of the chunk's rows in
// `tab` (built by the whole workgroup), then per round widen, RoPE,
// rotate and quantize into the wave's LDS region.
template <int TYPE, class Source>
__device__ inline void transform_rounds(const Source &s, const Chunk &c,
                                        const uint4 v[rounds_of(TYPE, true)], uint8_t *wl,
                                        float2 *tab, uint32_t wg0, uint32_t lane, bool build_tab) {
    constexpr int kRounds = rounds_of(TYPE, true);
    constexpr int GB = Fmt<TYPE>::GB;
    const uint32_t quad = lane >> 2;
    const uint32_t q = lane & 3u;
    const uint32_t half = s.n_rot / 2u;
    const uint32_t row0 = c.g0 / c.gpr;
    // Table row r holds pair j's (cos, sin) at position 2*(pl*((j%8)/2) +
    // j/8) + j%2, pl = half/8 lanes: a lane owning pairs 8m..8m+7 reads them
    // as four 16-byte chunks pl*u + m, u < 4, so in each read the lanes of
    // a half-head take consecutive chunks (no bank conflicts).
    const uint32_t pl = half / 8u;
    if (half != 0u && build_tab) {
        const uint32_t rows = (c.g0 + c.ng - 1u) / c.gpr - row0 + 1u;
        for (uint32_t i = threadIdx.x; i < rows * half; i += blockDim.x) {
            const uint32_t r = i / half;
            const uint32_t j = i - r * half;
            const float pos = static_cast<float>(c.pos0 + static_cast<int32_t>(row0 + r));
            float sn, cs;
            rope_sincos(pos * s.theta[j], sn, cs);
            tab[r * half + 2u * (pl * ((j & 7u) >> 1) + (j >> 3)) + (j & 1u)] = make_float2(cs, sn);
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
        const uint32_t gl = wg0 + 16u * r + quad;
        const bool valid = gl < c.ng;
        const uint32_t g = c.g0 + gl;
        const uint32_t row = g / c.gpr;
        const uint32_t col = g - row * c.gpr;
        const uint32_t d0 = (col * 32u + 8u * q) & (s.head_dim - 1u);  // first element in the head
        uint32_t h[8];
        unpack8(v[r], h);
        float x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            x[i] = half_bits_to_float(h[i]);
        }
        if (half != 0u) {
            const bool rot = d0 < s.n_rot;
            const bool first = d0 < half;
            float p[8];
            rope_partners(x, p, s.n_rot, lane, rot, first);
            if (rot && valid) {
                const uint32_t m = (first ? d0 : d0 - half) / 8u;
                const float4 *t = reinterpret_cast<const float4 *>(tab + (row - row0) * half);
                // first half (x0 = own, x1 = partner): own*c - partner*s;
                // second half (x0 = partner, x1 = own): own*c + partner*s
                const uint32_t flip = first ? 0x80000000u : 0u;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const float4 cs = t[pl * u + m];  // pairs 8m+2u (x, y), 8m+2u+1 (z, w)
                    const float p0 = p[2 * u] * cs.y;
                    const float p1 = p[2 * u + 1] * cs.w;
                    x[2 * u] = x[2 * u] * cs.x + __uint_as_float(__float_as_uint(p0) ^ flip);
                    x[2 * u + 1] = x[2 * u + 1] * cs.z + __uint_as_float(__float_as_uint(p1) ^ flip);
                }
            }
        }
        if (s.hadamard != 0u) {
            fwht_lanes(x, s.hadamard, s.hscale, lane);
        }
        quant_quarter_f<TYPE>(x, q, wl + (16u * r + quad) * GB, valid);
    }
}

// Quantize chunk `c` of `source` into its destination.  `lds` holds
// 4 * kWaveGroups groups of the type's layout; with XF the rows go through
// the source's transform and `tab` holds kTabMax cos/sin pairs.  The
// source's chunk_groups is chunk_groups_of(TYPE, XF).
template <int TYPE, class Source, bool XF>
__device__ inline void quant_chunk_body(const Source &source, const Chunk &c, uint8_t *lds,
                                        float2 *tab, bool build_tab) {
    constexpr int GB = Fmt<TYPE>::GB;
    constexpr int kRounds = rounds_of(TYPE, XF);
    constexpr int kWaveGroups = 16 * kRounds;
    constexpr int kChunkGroups = 4 * kWaveGroups;
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6;
    const uint32_t lane = tid & 63u;
    const uint32_t quad = lane >> 2;
    const uint32_t q = lane & 3u;
    const uint32_t wg0 = wave * kWaveGroups;
    uint8_t *wl = lds + wave * kWaveGroups * GB;

    // A full chunk of a contiguous source (every chunk but an operation's
    // last) needs neither the row/column split nor per-lane bounds: one
    // base address, 1 KiB apart per round, and no partial groups.
    const bool full_chunk = Source::kContiguous && c.ng == static_cast<uint32_t>(kChunkGroups);
    uint4 v[kRounds];
    if (full_chunk) {
        const uint8_t *base = c.src + static_cast<uint64_t>(c.g0 + wg0 + quad) * 64u + q * 16u;
#pragma unroll
        for (int r = 0; r < kRounds; ++r) {
            v[r] = load_stream16(base + r * 1024u);
        }
    } else {
#pragma unroll
        for (int r = 0; r < kRounds; ++r) {
            const uint32_t gl = wg0 + 16u * r + quad;
            v[r] = make_uint4(0u, 0u, 0u, 0u);
            if (gl < c.ng) {
                const uint32_t g = c.g0 + gl;
                const uint32_t row = g / c.gpr;
                const uint32_t col = g - row * c.gpr;
                const uint8_t *p = c.src + static_cast<uint64_t>(row) * c.src_stride + col * 64u + q * 16u;
                v[r] = load_stream16(p);
            }
        }
    }
    if constexpr (XF) {
        transform_rounds<TYPE>(source, c, v, wl, tab, wg0, lane, build_tab);
    } else if (full_chunk) {
#pragma unroll
        for (int r = 0; r < kRounds; ++r) {
            quant_quarter<TYPE>(v[r], q, wl + (16u * r + quad) * GB, true);
        }
    } else {
#pragma unroll
        for (int r = 0; r < kRounds; ++r) {
            const uint32_t gl = wg0 + 16u * r + quad;
            quant_quarter<TYPE>(v[r], q, wl + (16u * r + quad) * GB, gl < c.ng);
        }
    }
    // each wave reads back only the bytes it wrote itself
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    const uint32_t ngw = c.ng > wg0 ? min(static_cast<uint32_t>(kWaveGroups), c.ng - wg0) : 0u;
    const uint32_t nb = ngw * GB;
    uint8_t *dst = c.dst + static_cast<uint64_t>(c.g0 + wg0) * GB;
    // A slot whose groups are not a multiple of 8 (block_tokens x groups per
    // row) starts 2-byte aligned only: its bytes go out 2 at a time (groups
    // and slots are whole even-sized units, so every such address is even).
    const uint32_t full = (reinterpret_cast<uintptr_t>(dst) & 15u) == 0 ? (nb & ~15u) : 0u;
    for (uint32_t off = lane * 16u; off < full; off += 1024u) {
        // packed rows are read by attention later, not by this launch
        const u32x4_t w = *reinterpret_cast<const u32x4_t *>(wl + off);
        __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t *>(dst + off));
    }
    for (uint32_t off = full + lane * 2u; off < nb; off += 128u) {
        *reinterpret_cast<uint16_t *>(dst + off) = *reinterpret_cast<const uint16_t *>(wl + off);
    }
}

template <int TYPE, class Source, bool XF>
__device__ inline void quant_chunk(const Source &source, uint32_t c_index, uint8_t *lds,
                                   float2 *tab) {
    Chunk c;
    if (!source.chunk(c_index, c)) {
        return;  // uniform across the workgroup
    }
    quant_chunk_body<TYPE, Source, XF>(source, c, lds, tab, true);
}

// Workgroup chunk index `c` of a RoPE'd block source with layer grouping:
// the same rows of layer_group consecutive layers of one block.  Their
// positions, hence their cos/sin table, are the same, so the table is built
// once for all of them.  (A separate kernel instantiation: the layer loop
// costs registers that the other transformed sources do not pay.)
template <int TYPE>
__device__ inline void block_chunks(const BlockSource &s, uint32_t c, uint8_t *lds, float2 *tab) {
    const uint32_t groups = (s.n_layers + s.layer_group - 1u) / s.layer_group;
    const uint32_t og = c / s.chunks_per_op;
    const uint32_t sub = c - og * s.chunks_per_op;
    const uint32_t item = og / groups;
    const uint32_t l0 = (og - item * groups) * s.layer_group;
    const uint32_t l1 = min(s.n_layers, l0 + s.layer_group);
    for (uint32_t l = l0; l < l1; ++l) {
        Chunk ch;
        if (!s.chunk_at(item, l, sub, ch)) {
            return;  // uniform: no rows in this chunk for any layer
        }
        quant_chunk_body<TYPE, BlockSource, true>(s, ch, lds, tab, l == l0);
    }
}

// The RoPE table lives in dynamic LDS sized by the launch (rows a chunk
// touches x rotary pairs, at most kTabMax entries; 0 without RoPE), read
// as 16-byte chunks.
extern __shared__ float4 rope_tab4[];
#define rope_tab reinterpret_cast<float2 *>(rope_tab4)

// Chunk of workgroup `b` out of `n`.  Workgroups go to the 8 XCDs round-robin
// by id; in each group of 8 * kXcdTile chunks, XCD x takes kXcdTile
// consecutive chunks (whole operations: a (block, layer) run of 128 tokens
// x 1024 elements is 4 to 16 chunks), so the pages of an operation are
// translated by one XCD only, while the chunks in flight on the chip stay
// one contiguous window.  The tail of fewer than 8 * kXcdTile chunks keeps
// the identity order.  A bijection on [0, n).
constexpr uint32_t kXcdTile = 64;
__device__ inline uint32_t xcd_chunk(uint32_t b, uint32_t n) {
    constexpr uint32_t G = 8u * kXcdTile;
    if (b >= n - n % G) {
        return b;
    }
    const uint32_t r = b % G;
    return (b - r) + (r & 7u) * kXcdTile + (r >> 3);
}

// LDS staging bytes of a workgroup: 4 waves x 16 * R groups of the format.
template <int TYPE, bool XF>
constexpr int stage_bytes() {
    return 4 * 16 * rounds_of(TYPE, XF) * Fmt<TYPE>::GB;
}

template <int TYPE, class Source, bool XF, bool GROUP>
__global__ __launch_bounds__(256) void quant_scatter_kernel(Source arg, ArgTables t) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[stage_bytes<TYPE, XF>()];
    Source source = arg;
    source.bind(t);
    const uint32_t c = xcd_chunk(blockIdx.x, gridDim.x);
    if constexpr (GROUP) {
        block_chunks<TYPE>(source, c, lds, rope_tab);
    } else {
        quant_chunk<TYPE, Source, XF>(source, c, lds, rope_tab);
    }
}

// K and V of a block job in one launch: chunks [0, n_k) are K, the rest V
// (the branch is uniform per workgroup).
template <int TK, int TV, bool XF, bool GROUP>
__global__ __launch_bounds__(256) void quant_scatter_kv_kernel(BlockSource ak, BlockSource av, uint32_t n_k,
                                                               ArgTables t) {
    BlockSource sk = ak, sv = av;
    sk.bind(t);
    sv.bind(t);
    constexpr int SB = stage_bytes<TK, XF>() > stage_bytes<TV, XF>() ? stage_bytes<TK, XF>()
                                                                     : stage_bytes<TV, XF>();
    __shared__ __attribute__((aligned(16))) uint8_t lds[SB];
    const uint32_t c = xcd_chunk(blockIdx.x, gridDim.x);
    if (c < n_k) {
        if constexpr (GROUP) {
            block_chunks<TK>(sk, c, lds, rope_tab);
        } else {
            quant_chunk<TK, BlockSource, XF>(sk, c, lds, rope_tab);
        }
    } else {
        quant_chunk<TV, BlockSource, XF>(sv, c - n_k, lds, rope_tab);
    }
}

// ------------------------------------------ transformed rows, 64 per lane
//
// The transformed path above gives each lane 8 elements, so most butterfly
// stages and every quantization group span lanes, and each cross-lane step
// costs an exchange, a sign and an add per element.  This path gives each
// lane 64 consecutive elements of a row (two quantization groups) and a
// wave a unit of 4096 consecutive elements of an operation; a workgroup
// takes one unit of one block for every layer, wave w the layers w, w + 4,
// ... (four workgroups per CU hide each other's load latency).  Loads
// stay coalesced (16 bytes per lane, 1 KiB per wave-wide load) and are
// redistributed through the wave's LDS with a lane stride of 136 bytes
// (8-byte halves of consecutive lanes fall on distinct banks on both sides,
// and every address is one base plus an immediate offset).  Then:
//  - Hadamard spans 1 .. 32 are butterflies inside the lane; spans 64, 128
//    and 256 pair lane l with l ^ 1, ^ 2, ^ 4.  A cross-lane stage is one
//    fused multiply-add per element, y = fma(partner, t, own) with t = -1
//    in the lane that holds the upper element: fma(p, +-1, y) rounds y +- p
//    once, as the IEEE sum does, and the upper lane then holds the negation
//    of its value (round to nearest even is odd-symmetric).  After the
//    stages a lane holds sigma * x with sigma = (-1)^(its cross-lane bits),
//    folded into the quantizer: the scale reads |x| and the codes are
//    y * (sigma * id) = x * id.  Only the sign of an exact zero can differ,
//    which q8_0, q4_0 and q5_0 never show; F16 rows with cross-lane stages
//    take the path above.
//  - A Hadamard scale that is a power of two (widths 64 and 256: 1/8,
//    1/16) is not applied to the elements.  Every nonzero value of the
//    transform lies between 2^-100 and 2^40 in magnitude (f16 inputs,
//    products with cos/sin rounded to 24 bits, rounded sums of those), so
//    scaling by a power of two commutes with every rounded operation; the
//    quantizer scales amax (exactly) and multiplies id by the scale
//    (exactly) instead.  1/sqrtf(128) and 1/sqrtf(512) are inexact and
//    scale the elements first, as the reference does.
//  - RoPE (n_rot 128 and 256): a rotary pair lies in lanes l and
//    l ^ n_rot/128, and an element becomes fma(partner * sin, t, own * cos),
//    t = -1 in the first half: the two rounded products and the one rounded
//    sum of x0*c - x1*s and x0*s + x1*c.  Partners (here and for the
//    butterflies) come through ds_bpermute, off the vector ALU.
//  - The cos/sin table of the unit's rows is built once per workgroup for
//    all the layers.
constexpr uint32_t kX64Lane = 136;              // LDS bytes per lane: 128 + 8
constexpr uint32_t kX64Wave = 64u * kX64Lane;   // LDS bytes of one wave
constexpr uint32_t kX64Groups = 128; // groups of 32 elements in a unit

// cos/sin table of rotary pairs (n_rot = 2 * half, half 64 or 128) in
// 16-byte units of two pairs (c_j, s_j, c_j+1, s_j+1).  A lane reads P = 64
// consecutive pairs; a row holds half / P runs of P/2 units, each followed
// by one unused unit, so that the rows and runs one wave-wide read touches
// fall on distinct banks.
struct X64Tab {
    uint32_t P, JS, RS;  // pairs per run, units per run (+1), units per row
};
__host__ __device__ inline X64Tab x64_tab_geom(uint32_t half) {
    const uint32_t P = half < 64u ? half : 64u;
    const uint32_t JS = P / 2u + 1u;
    return {P, JS, (half / P) * JS};
}

// A unit's 16-byte loads: load k of lane i holds elements 512k + 8i .. +7
// of the 4096, owned by lane 8k + i/8.  Loads owned by lanes past the
// operation's end are not issued.
__device__ inline void x64_load(const Chunk &c, uint32_t lane, uint32_t nvl, uint4 v[8]) {
    const uint8_t *base = c.src + static_cast<uint64_t>(c.g0) * 64u + lane * 16u;
    if (nvl == 64u) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            v[k] = load_stream16(base + k * 1024);
        }
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            v[k] = make_uint4(0u, 0u, 0u, 0u);
            if (8u * k + (lane >> 3) < nvl) {
                v[k] = load_stream16(base + k * 1024);
            }
        }
    }
}

__device__ inline void wave_lds_order() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The value of lane ^ m (m uniform) through ds_bpermute, on the LDS pipe.
__device__ inline float x64_partner(float v, uint32_t src_addr) {
    return __int_as_float(__builtin_amdgcn_ds_bpermute(static_cast<int>(src_addr), __float_as_int(v)));
}

// v_fma_mix_f32 on the f16 halves of a packed pair: an f16 operand is
// widened exactly, so fma(lo, 1, hi) rounds lo + hi once (the IEEE sum of
// the widened values), fma(hi, -1, lo) is lo - hi and fma(h, c, -0) is the
// product h * c rounded once (-0 keeps the sign of a zero product).  The
// widening then costs no instruction of its own.
__device__ inline float mix_sum(uint32_t w) {
    float r;
    asm("v_fma_mix_f32 %0, %1, 1.0, %1 op_sel:[0,0,1] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(w));
    return r;
}
__device__ inline float mix_diff(uint32_t w) {
    float r;
    asm("v_fma_mix_f32 %0, %1, -1.0, %1 op_sel:[1,0,0] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(w));
    return r;
}
template <int HI>
__device__ inline float mix_mul(uint32_t w, float c, float nz) {
    float r;
    if constexpr (HI) {
        asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(c), "v"(nz));
    } else {
        asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(c), "v"(nz));
    }
    return r;
}

// RoPE of pairs across lanes (src_addr = 4 * the partner lane) straight from
// the packed f16 words (word u: elements 2u, 2u + 1), one exchange per word.
__device__ inline void x64_rope_f16(float x[64], const uint32_t w[32], const float4 *t, float tr,
                                    uint32_t src_addr) {
    const float nz = -0.0f;
#pragma unroll
    for (int u = 0; u < 32; ++u) {
        const float4 cs = t[u];  // pairs of elements 2u (x: cos, y: sin) and 2u + 1 (z, w)
        const uint32_t pw = static_cast<uint32_t>(
            __builtin_amdgcn_ds_bpermute(static_cast<int>(src_addr), static_cast<int>(w[u])));
        const float p0 = mix_mul<0>(pw, cs.y, nz);
        const float p1 = mix_mul<1>(pw, cs.w, nz);
        const float a0 = mix_mul<0>(w[u], cs.x, nz);
        const float a1 = mix_mul<1>(w[u], cs.z, nz);
        x[2 * u] = __builtin_fmaf(p0, tr, a0);
        x[2 * u + 1] = __builtin_fmaf(p1, tr, a1);
    }
}

// vmax of q4_0 / q5_0 (first element of largest magnitude, ggml's strict
// scan) of group y[0..31] as held: +0 for an all-zero group.
__device__ inline float x64_vmax(const float *y) {
    float mx = 0.0f, mn = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        mx = fmaxf(mx, y[i]);
        mn = fminf(mn, y[i]);
    }
    const float a = fmaxf(mx, -mn);
    if (a == 0.0f) {
        return 0.0f;
    }
    if (mx == a && -mn == a) {  // both signs reach amax: the first one wins
        uint32_t neg = 0u;
#pragma unroll
        for (int i = 31; i >= 0; --i) {
            if (fabsf(y[i]) == a) {
                neg = __float_as_uint(y[i]) >> 31;
            }
        }
        return neg ? -a : a;
    }
    return mx == a ? a : -a;
}

// Codes of one q4_0 / q5_0 group as bytes: word m holds codes 4m .. 4m+3
// (lo) and 16+4m .. 16+4m+3 (hi).
template <int TOP>
__device__ inline void x64_trunc_codes(const float *y, float idf, float bias, uint32_t lo[4],
                                       uint32_t hi[4]) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        lo[m] = 0u;
        hi[m] = 0u;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            lo[m] |= trunc_code<TOP>(y[4 * m + b], idf, bias) << (8 * b);
            hi[m] |= trunc_code<TOP>(y[16 + 4 * m + b], idf, bias) << (8 * b);
        }
    }
}

// Quantize one group (32 values y held as sigma * x / scale; f = sigma *
// scale, sf = scale) into its f16 scale bits and P payload words.
template <int TYPE> struct X64Q;

template <> struct X64Q<KVMEM_TYPE_Q8_0> {
    static constexpr int P = 8;
    __device__ static inline uint32_t group(const float *y, float f, float sf, uint32_t w[P]) {
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            a = fmaxf(a, fabsf(y[i]));
        }
        const float d = scale_div127(a * sf);
        const float id = d != 0.0f ? scale_recip(d) : 0.0f;
        const float idf = id * f;
#pragma unroll
        for (int m = 0; m < P; ++m) {
            w[m] = 0u;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                w[m] |= (static_cast<uint32_t>(round_q8(y[4 * m + b] * idf)) & 0xffu) << (8 * b);
            }
        }
        return float_to_half_bits(d);
    }
};

template <> struct X64Q<KVMEM_TYPE_Q4_0> {
    static constexpr int P = 4;
    __device__ static inline uint32_t group(const float *y, float f, float, uint32_t w[P]) {
        const float vm = x64_vmax(y);
        const float d = (vm != 0.0f ? vm * f : 0.0f) * -0.125f;  // vmax of x / -8, both exact
        const float id = d != 0.0f ? scale_recip(d) : 0.0f;
        uint32_t lo[4], hi[4];
        x64_trunc_codes<15>(y, id * f, 8.5f, lo, hi);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            w[m] = lo[m] | (hi[m] << 4);
        }
        return float_to_half_bits(d);
    }
};

template <> struct X64Q<KVMEM_TYPE_Q5_0> {
    static constexpr int P = 5;
    __device__ static inline uint32_t group(const float *y, float f, float, uint32_t w[P]) {
        const float vm = x64_vmax(y);
        const float d = (vm != 0.0f ? vm * f : 0.0f) * -0.0625f;  // vmax of x / -16, both exact
        const float id = d != 0.0f ? scale_recip(d) : 0.0f;
        uint32_t lo[4], hi[4];
        x64_trunc_codes<31>(y, id * f, 16.5f, lo, hi);
        uint32_t qh = 0u;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            qh |= (bit4_of_bytes(lo[m]) << (4 * m)) | (bit4_of_bytes(hi[m]) << (16 + 4 * m));
            w[1 + m] = (lo[m] & 0x0f0f0f0fu) | ((hi[m] & 0x0f0f0f0fu) << 4);
        }
        w[0] = qh;
        return float_to_half_bits(d);
    }
};

// The lane's two groups in ggml's byte layout as 2 * GB / 4 words (GB is 2
// mod 4: the second group starts two bytes into a word).
template <int TYPE>
__device__ inline void x64_quant_lane(const float x[64], float f, float sf, uint32_t *dst) {
    if constexpr (TYPE == KVMEM_TYPE_F16) {
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            dst[i] = float_to_half_bits(x[2 * i]) | (float_to_half_bits(x[2 * i + 1]) << 16);
        }
    } else {
        constexpr int P = X64Q<TYPE>::P;
        uint32_t w0[P], w1[P];
        const uint32_t d0 = X64Q<TYPE>::group(x, f, sf, w0);
        const uint32_t d1 = X64Q<TYPE>::group(x + 32, f, sf, w1);
        dst[0] = d0 | (w0[0] << 16);
#pragma unroll
        for (int m = 1; m < P; ++m) {
            dst[m] = __builtin_amdgcn_alignbit(w0[m], w0[m - 1], 16);
        }
        dst[P] = (w0[P - 1] >> 16) | (d1 << 16);
#pragma unroll
        for (int m = 0; m < P; ++m) {
            dst[P + 1 + m] = w1[m];
        }
    }
}

// Workgroup `c` of a block source on this path: unit `sub` (groups g0 ..
// g0+ng, ng <= 128) of one block, wave w taking layers w, w + 4, ...
template <int TYPE>
__device__ inline void x64_unit_layers(const BlockSource &s, uint32_t c, uint8_t *lds, uint8_t *tab) {
    constexpr int GB = Fmt<TYPE>::GB;
    const uint32_t item = c / s.chunks_per_op;
    const uint32_t sub = c - item * s.chunks_per_op;
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
    const uint32_t lane = tid & 63u;
    // the item's fields, read once (uniform): block, slot, tokens, position
    const uint32_t block = s.items[4 * item + 0];
    const uint32_t slot = s.items[4 * item + 1];
    Chunk ch;
    ch.pos0 = static_cast<int32_t>(s.items[4 * item + 3]);
    ch.gpr = s.gpr;
    ch.src_stride = s.gpr * 64u;
    ch.g0 = sub * kX64Groups;
    const uint32_t total = s.items[4 * item + 2] * s.gpr;
    if (ch.g0 >= total) {
        return;  // uniform: no rows in this unit
    }
    ch.ng = min(kX64Groups, total - ch.g0);
    const uint8_t *src0 = s.base + block * s.block_stride;
    const uint64_t dst_off = static_cast<uint64_t>(slot) * s.block_tokens * s.row_bytes;
    const uint32_t nvl = min(64u, ch.ng / 2u);  // lanes with elements (ng is even)
    uint8_t *wl = lds + wave * kX64Wave;

    // the lane's place: row, offset in its head
    const uint32_t E = s.gpr * 32u;
    const uint32_t e = (ch.g0 + 2u * lane) * 32u;
    const uint32_t row = e / E;
    const uint32_t d0 = (e - row * E) & (s.head_dim - 1u);
    const uint32_t row0 = ch.g0 / ch.gpr;
    const uint32_t half = s.n_rot / 2u;
    const X64Tab tg = x64_tab_geom(half);
    if (half != 0u) {
        const uint32_t rows = (ch.g0 + ch.ng - 1u) / ch.gpr - row0 + 1u;
        for (uint32_t i = tid; i < rows * half; i += blockDim.x) {
            const uint32_t r = i / half;
            const uint32_t j = i - r * half;
            const float pos = static_cast<float>(ch.pos0 + static_cast<int32_t>(row0 + r));
            float sn, cs;
            rope_sincos(pos * s.theta[j], sn, cs);
            const uint32_t off = (r * tg.RS + (j / tg.P) * tg.JS + (j % tg.P) / 2u) * 16u + (j & 1u) * 8u;
            *reinterpret_cast<float2 *>(tab + off) = make_float2(cs, sn);
        }
        __syncthreads();
    }
    // RoPE (n_rot 128 or 256): the pair of element d0 + k is element
    // d0 + k +- half of lane ^ half/64, the cos/sin of pairs j0 .. j0 + 63
    const bool first = d0 < half;
    const bool rot = lane < nvl && d0 < s.n_rot;
    const uint32_t j0 = first ? d0 : d0 - half;
    const float4 *trow = reinterpret_cast<const float4 *>(tab + ((row - row0) * tg.RS + (j0 / 64u) * tg.JS) * 16u);
    const float tr = first ? -1.0f : 1.0f;
    const uint32_t rope_src = 4u * (lane ^ (half / 64u));
    // cross-lane butterflies: stages on lane bits 0 .. nx-1, and the sign
    // they leave
    const uint32_t W = s.hadamard;
    const uint32_t nx = W >= 512u ? 3u : W >= 256u ? 2u : W >= 128u ? 1u : 0u;
    const float sigma = (__popc(lane & ((1u << nx) - 1u)) & 1u) ? -1.0f : 1.0f;
    // a power-of-two scale is carried into the quantizer (never for F16)
    const bool fold = TYPE != KVMEM_TYPE_F16 && (__float_as_uint(s.hscale) & 0x007fffffu) == 0u;
    const float sf = (W != 0u && fold) ? s.hscale : 1.0f;
    const float f = sigma * sf;
    // without RoPE the first operation is the Hadamard's span-1 butterfly
    // (scale carried) or its scale
    const bool first_sum = half == 0u && W != 0u && fold;
    const bool first_scale = half == 0u && W != 0u && !fold;
    // LDS places: chunk lane % 8 of load k belongs to lane 8k + lane/8
    uint8_t *wr = wl + (lane >> 3) * kX64Lane + (lane & 7u) * 16u;
    const uint8_t *rd = wl + lane * kX64Lane;

    for (uint32_t l = wave; l < s.n_layers; l += 4u) {
        ch.src = src0 + l * s.layer_stride;  // the same rows of layer l
        ch.dst = const_cast<uint8_t *>(s.layer_dst[l]) + dst_off;
        uint4 v[8];
        x64_load(ch, lane, nvl, v);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            uint2 *q = reinterpret_cast<uint2 *>(wr + k * 8u * kX64Lane);
            q[0] = make_uint2(v[k].x, v[k].y);
            q[1] = make_uint2(v[k].z, v[k].w);
        }
        wave_lds_order();
        uint32_t w[32];  // packed f16 pairs: word m holds elements 2m, 2m + 1
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint2 lo = reinterpret_cast<const uint2 *>(rd + 16u * j)[0];
            const uint2 hi = reinterpret_cast<const uint2 *>(rd + 16u * j)[1];
            w[4 * j + 0] = lo.x;
            w[4 * j + 1] = lo.y;
            w[4 * j + 2] = hi.x;
            w[4 * j + 3] = hi.y;
        }
        // the first operation on each element widens it
        float x[64];
        if (half != 0u && rot) {
            x64_rope_f16(x, w, trow, tr, rope_src);
        } else if (first_sum) {  // Hadamard span 1 with the scale carried to the quantizer
#pragma unroll
            for (int m = 0; m < 32; ++m) {
                x[2 * m] = mix_sum(w[m]);
                x[2 * m + 1] = mix_diff(w[m]);
            }
        } else if (first_scale) {  // the inexact Hadamard scale
#pragma unroll
            for (int m = 0; m < 32; ++m) {
                x[2 * m] = mix_mul<0>(w[m], s.hscale, -0.0f);
                x[2 * m + 1] = mix_mul<1>(w[m], s.hscale, -0.0f);
            }
        } else {
#pragma unroll
            for (int m = 0; m < 32; ++m) {
                x[2 * m] = half_bits_to_float(w[m] & 0xffffu);
                x[2 * m + 1] = half_bits_to_float(w[m] >> 16);
            }
        }
        if (W != 0u) {
            if (!fold && half != 0u) {
#pragma unroll
                for (int i = 0; i < 64; ++i) {
                    x[i] = x[i] * s.hscale;
                }
            }
            if (!first_sum) {
#pragma unroll
                for (int i = 0; i < 64; i += 2) {
                    const float a = x[i];
                    const float b = x[i + 1];
                    x[i] = a + b;
                    x[i + 1] = a - b;
                }
            }
#pragma unroll
            for (int h = 2; h < 64; h <<= 1) {
#pragma unroll
                for (int i = 0; i < 64; i += 2 * h) {
#pragma unroll
                    for (int j = 0; j < h; ++j) {
                        const float a = x[i + j];
                        const float b = x[i + j + h];
                        x[i + j] = a + b;
                        x[i + j + h] = a - b;
                    }
                }
            }
            for (uint32_t st = 0; st < nx; ++st) {
                // y = own + t * partner, t = -1 where the lane holds the upper element
                const uint32_t src = 4u * (lane ^ (1u << st));
                const float t = ((lane >> st) & 1u) ? -1.0f : 1.0f;
#pragma unroll
                for (int i = 0; i < 64; ++i) {
                    x[i] = __builtin_fmaf(x64_partner(x[i], src), t, x[i]);
                }
            }
        }
        wave_lds_order();  // every lane's input is read before outputs overwrite it
        x64_quant_lane<TYPE>(x, f, sf, reinterpret_cast<uint32_t *>(wl + lane * (2u * GB)));
        wave_lds_order();
        const uint32_t nb = nvl * 2u * GB;
        uint8_t *out = ch.dst + static_cast<uint64_t>(ch.g0) * GB;
        if ((reinterpret_cast<uintptr_t>(out) & 15u) == 0) {
            const uint32_t full = nb & ~15u;
            for (uint32_t off = lane * 16u; off < full; off += 1024u) {
                const u32x4_t w = *reinterpret_cast<const u32x4_t *>(wl + off);
                __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t *>(out + off));
            }
            for (uint32_t off = full + lane * 4u; off < nb; off += 256u) {
                *reinterpret_cast<uint32_t *>(out + off) = *reinterpret_cast<const uint32_t *>(wl + off);
            }
        } else {
            // a slot of a group count not a multiple of 8 starts 2-byte aligned only
            for (uint32_t off = lane * 2u; off < nb; off += 128u) {
                *reinterpret_cast<uint16_t *>(out + off) = *reinterpret_cast<const uint16_t *>(wl + off);
            }
        }
        wave_lds_order();  // the copy-out reads finish before the next layer's rows land
    }
}

template <int TYPE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void x64_kernel(BlockSource a,
                                                                                            ArgTables t) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[4 * kX64Wave];
    BlockSource s = a;
    s.bind(t);
    x64_unit_layers<TYPE>(s, xcd_chunk(blockIdx.x, gridDim.x), lds, reinterpret_cast<uint8_t *>(rope_tab4));
}

template <int TK, int TV>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void x64_kv_kernel(BlockSource ak, BlockSource av, uint32_t n_k, ArgTables t) {
    BlockSource sk = ak, sv = av;
    sk.bind(t);
    sv.bind(t);
    __shared__ __attribute__((aligned(16))) uint8_t lds[4 * kX64Wave];
    const uint32_t c = xcd_chunk(blockIdx.x, gridDim.x);
    uint8_t *tab = reinterpret_cast<uint8_t *>(rope_tab4);
    if (c < n_k) {
        x64_unit_layers<TK>(sk, c, lds, tab);
    } else {
        x64_unit_layers<TV>(sv, c - n_k, lds, tab);
    }
}

// Dynamic LDS bytes of the RoPE table for chunks of `s`.
template <class Source>
size_t rope_tab_bytes(const Source &s) {
    return s.n_rot ? sizeof(float2) * chunk_rows_of(s.gpr, s.chunk_groups) * (s.n_rot / 2) : 0;
}

template <class Source, bool XF, bool GROUP>
bool launch_quant_x(kvmem_hip_ctx *ctx, int type, uint32_t n_chunks, const Source &s, const ArgTables &args) {
    if (injected_fail(ctx, KVMEM_HIP_FAIL_LAUNCH, "stage-in kernel launch")) {
        return false;
    }
    size_t tb = 0;
    if constexpr (XF) {
        tb = rope_tab_bytes(s);
    }
    switch (type) {
        case KVMEM_TYPE_Q8_0:
            ctx_launch(ctx, quant_scatter_kernel<KVMEM_TYPE_Q8_0, Source, XF, GROUP>, dim3(n_chunks), dim3(256), static_cast<uint32_t>(tb), s, args);
            break;
        case KVMEM_TYPE_Q4_0:
            ctx_launch(ctx, quant_scatter_kernel<KVMEM_TYPE_Q4_0, Source, XF, GROUP>, dim3(n_chunks), dim3(256), static_cast<uint32_t>(tb), s, args);
            break;
        case KVMEM_TYPE_Q5_0:
            ctx_launch(ctx, quant_scatter_kernel<KVMEM_TYPE_Q5_0, Source, XF, GROUP>, dim3(n_chunks), dim3(256), static_cast<uint32_t>(tb), s, args);
            break;
        case KVMEM_TYPE_F16:
            ctx_launch(ctx, quant_scatter_kernel<KVMEM_TYPE_F16, Source, XF, GROUP>, dim3(n_chunks), dim3(256), static_cast<uint32_t>(tb), s, args);
            break;
        default:
            fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "stage-in: unsupported type");
            return false;
    }
    return hip_ok(ctx, hipGetLastError(), "stage-in kernel launch");
}

static const ArgTables kNoArgTables{};

bool launch_quant(kvmem_hip_ctx *ctx, int type, uint32_t n_chunks, const OpListSource &s) {
    return n_chunks == 0 || launch_quant_x<OpListSource, false, false>(ctx, type, n_chunks, s, kNoArgTables);
}

bool launch_quant(kvmem_hip_ctx *ctx, int type, uint32_t n_chunks, const BlockSource &s, bool xf,
                  const ArgTables &args) {
    if (n_chunks == 0) {
        return true;
    }
    if (!xf) {
        return launch_quant_x<BlockSource, false, false>(ctx, type, n_chunks, s, args);
    }
    return s.layer_group > 1u ? launch_quant_x<BlockSource, true, true>(ctx, type, n_chunks, s, args)
                              : launch_quant_x<BlockSource, true, false>(ctx, type, n_chunks, s, args);
}

template <int TK, bool XF, bool GROUP>
bool launch_kv_v(kvmem_hip_ctx *ctx, int tv, uint32_t grid, const BlockSource &sk,
                 const BlockSource &sv, uint32_t n_k, const ArgTables &args) {
    if (injected_fail(ctx, KVMEM_HIP_FAIL_LAUNCH, "stage-in K/V kernel launch")) {
        return false;
    }
    const size_t tb = XF ? rope_tab_bytes(sk) : 0;  // only K is RoPE'd
    switch (tv) {
        case KVMEM_TYPE_Q8_0:
            ctx_launch(ctx, quant_scatter_kv_kernel<TK, KVMEM_TYPE_Q8_0, XF, GROUP>, dim3(grid), dim3(256), static_cast<uint32_t>(tb), sk, sv, n_k, args);
            break;
        case KVMEM_TYPE_Q4_0:
            ctx_launch(ctx, quant_scatter_kv_kernel<TK, KVMEM_TYPE_Q4_0, XF, GROUP>, dim3(grid), dim3(256), static_cast<uint32_t>(tb), sk, sv, n_k, args);
            break;
        case KVMEM_TYPE_Q5_0:
            ctx_launch(ctx, quant_scatter_kv_kernel<TK, KVMEM_TYPE_Q5_0, XF, GROUP>, dim3(grid), dim3(256), static_cast<uint32_t>(tb), sk, sv, n_k, args);
            break;
        case KVMEM_TYPE_F16:
            ctx_launch(ctx, quant_scatter_kv_kernel<TK, KVMEM_TYPE_F16, XF, GROUP>, dim3(grid), dim3(256), static_cast<uint32_t>(tb), sk, sv, n_k, args);
            break;
        default:
            fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "stage-in: unsupported V type");
            return false;
    }
    return hip_ok(ctx, hipGetLastError(), "stage-in K/V kernel launch");
}

template <bool XF, bool GROUP>
bool launch_quant_kv_x(kvmem_hip_ctx *ctx, int tk, int tv, uint32_t n_k, uint32_t n_v,
                       const BlockSource &sk, const BlockSource &sv, const ArgTables &args) {
    const uint32_t grid = n_k + n_v;
    switch (tk) {
        case KVMEM_TYPE_Q8_0: return launch_kv_v<KVMEM_TYPE_Q8_0, XF, GROUP>(ctx, tv, grid, sk, sv, n_k, args);
        case KVMEM_TYPE_Q4_0: return launch_kv_v<KVMEM_TYPE_Q4_0, XF, GROUP>(ctx, tv, grid, sk, sv, n_k, args);
        case KVMEM_TYPE_Q5_0: return launch_kv_v<KVMEM_TYPE_Q5_0, XF, GROUP>(ctx, tv, grid, sk, sv, n_k, args);
        case KVMEM_TYPE_F16: return launch_kv_v<KVMEM_TYPE_F16, XF, GROUP>(ctx, tv, grid, sk, sv, n_k, args);
        default:
            fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "stage-in: unsupported K type");
            return false;
    }
}

// The K source groups layers when it is RoPE'd (layer_group > 1); V never is.
bool launch_quant_kv(kvmem_hip_ctx *ctx, int tk, int tv, uint32_t n_k, uint32_t n_v,
                     const BlockSource &sk, const BlockSource &sv, bool xf, const ArgTables &args) {
    if (n_k + n_v == 0) {
        return true;
    }
    if (!xf) {
        return launch_quant_kv_x<false, false>(ctx, tk, tv, n_k, n_v, sk, sv, args);
    }
    return sk.layer_group > 1u ? launch_quant_kv_x<true, true>(ctx, tk, tv, n_k, n_v, sk, sv, args)
                               : launch_quant_kv_x<true, false>(ctx, tk, tv, n_k, n_v, sk, sv, args);
}

static bool aligned16(const void *p) {
    return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

static int check_pool(kvmem_hip_ctx *ctx, const kvmem_hip_pool *pool, uint32_t n_layers,
                      uint32_t block_tokens, uint32_t ek, uint32_t ev, bool want_v) {
    if (!pool || !pool->k_layers) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "pool: null");
    }
    if (pool->n_layers != n_layers || pool->block_tokens != block_tokens ||
        pool->n_embd_k != ek || (want_v && pool->n_embd_v != ev)) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "pool: geometry does not match the history");
    }
    if (!kvmem_hip_quant_ok(pool->type_k) || (want_v && !kvmem_hip_quant_ok(pool->type_v))) {
        return fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "pool: unsupported cache type");
    }
    for (uint32_t l = 0; l < n_layers; ++l) {
        if (!pool->k_layers[l] || !aligned16(pool->k_layers[l]) ||
            (want_v && (!pool->v_layers[l] || !aligned16(pool->v_layers[l])))) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID, "pool: layer pointer null or not 16-byte aligned");
        }
    }
    return KVMEM_HIP_OK;
}

// A pool's transform, checked and resolved per kind.
struct XfParams {
    bool on = false;
    bool lane64 = false;  // the 64-elements-per-lane kernels take the job
    uint32_t head_dim = 32;
    uint32_t n_rot = 0;
    uint32_t had_k = 0;
    uint32_t had_v = 0;
    float hscale_k = 1.0f;
    float hscale_v = 1.0f;
};

// Rows of n_embd elements that one transformed chunk can touch.
static uint32_t chunk_rows(uint32_t n_embd, int type) {
    return chunk_rows_of(n_embd / 32, chunk_groups_of(type, true));
}

static bool pow2_in(uint32_t x, uint32_t lo, uint32_t hi) {
    return x >= lo && x <= hi && (x & (x - 1)) == 0;
}

static int resolve_xf(kvmem_hip_ctx *ctx, const kvmem_hip_pool *pool, uint32_t ek, uint32_t ev,
                      bool want_v, XfParams &out) {
    out = XfParams{};
    const kvmem_hip_transform *xf = pool->xf;
    if (!xf || (xf->n_rot == 0 && xf->hadamard_k == 0 && (xf->hadamard_v == 0 || !want_v))) {
        return KVMEM_HIP_OK;
    }
    const uint32_t D = xf->head_dim;
    if (!pow2_in(D, 64, 512) || ek % D != 0 || (want_v && xf->hadamard_v && ev % D != 0)) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID,
                    "transform: head_dim must be 64, 128, 256 or 512 and divide the row");
    }
    if (xf->n_rot && (xf->n_rot % 16 != 0 || xf->n_rot > D || !xf->theta)) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID,
                    "transform: n_rot must be a multiple of 16 up to head_dim, with theta");
    }
    if (xf->n_rot && chunk_rows(ek, pool->type_k) * (xf->n_rot / 2) > static_cast<uint32_t>(kTabMax)) {
        return fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "transform: rows too narrow for the RoPE table");
    }
    for (uint32_t w : {xf->hadamard_k, want_v ? xf->hadamard_v : 0u}) {
        if (w && (!pow2_in(w, 64, 512) || D % w != 0)) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID,
                        "transform: Hadamard width must be 64..512, a power of two dividing head_dim");
        }
    }
    out.on = true;
    out.head_dim = D;
    out.n_rot = xf->n_rot;
    out.had_k = xf->hadamard_k;
    out.had_v = want_v ? xf->hadamard_v : 0u;
    // the reference's scale, 1.0f / sqrtf((float) nrot) (stagein.cu:557)
    out.hscale_k = out.had_k ? 1.0f / sqrtf(static_cast<float>(out.had_k)) : 1.0f;
    out.hscale_v = out.had_v ? 1.0f / sqrtf(static_cast<float>(out.had_v)) : 1.0f;
    // The 64-elements-per-lane kernels hold a rotary pair in lanes l and
    // l ^ n_rot/128 (n_rot 128, 256), and F16 rows only without cross-lane
    // butterflies (width 64); other shapes take the 8-elements-per-lane
    // kernels.
    const uint32_t half = out.n_rot / 2;
    out.lane64 = (half == 0 || half == 64 || half == 128) &&
                 ek % 64 == 0 && (!want_v || ev % 64 == 0) &&
                 (pool->type_k != KVMEM_TYPE_F16 || out.had_k <= 64) &&
                 (!want_v || pool->type_v != KVMEM_TYPE_F16 || out.had_v <= 64);
    return KVMEM_HIP_OK;
}

// One upload holding a block job's device tables: the pool's per-layer
// pointers (K at [0, L), V at [L, 2L)), the items ([n][4] u32: block, slot,
// tokens, position of token 0) and the RoPE frequencies.  A single upload
// per call keeps them inside one upload-ring slot for as long as the
// call's kernels need them.
struct JobTables {
    LaunchTables tables;  // [2L] layer pointers (K, then V), the items, the RoPE frequencies
    uint32_t items_off = 0;
    uint32_t theta_off = 0;
};

static bool stage_block_job(kvmem_hip_ctx *ctx, const kvmem_hip_pool *pool, bool want_v,
                            const std::vector<uint32_t> &items, const XfParams &xp, JobTables &out) {
    const size_t L = pool->n_layers;
    const size_t n_theta = xp.n_rot / 2;
    const size_t words = items.size() + n_theta;  // 4-byte words after the pointers
    std::vector<uint64_t> buf(2 * L + (words + 1) / 2, 0);
    for (size_t l = 0; l < L; ++l) {
        buf[l] = reinterpret_cast<uint64_t>(pool->k_layers[l]);
        buf[L + l] = want_v ? reinterpret_cast<uint64_t>(pool->v_layers[l]) : 0;
    }
    uint8_t *tail = reinterpret_cast<uint8_t *>(buf.data() + 2 * L);
    std::memcpy(tail, items.data(), items.size() * sizeof(uint32_t));
    if (n_theta) {
        std::memcpy(tail + items.size() * sizeof(uint32_t), pool->xf->theta, n_theta * sizeof(float));
    }
    out.items_off = static_cast<uint32_t>(2 * L * sizeof(uint64_t));
    out.theta_off = static_cast<uint32_t>(out.items_off + items.size() * sizeof(uint32_t));
    return stage_tables(ctx, buf.data(), buf.size() * sizeof(uint64_t), out.tables, "stage-in job tables");
}

// Position of token 0 of staged block i (item order of the call).
static uint32_t item_pos0(const kvmem_hip_pool *pool, const uint32_t *block_ids, uint32_t i,
                          uint32_t block_tokens) {
    if (pool->xf && pool->xf->pos0) {
        return static_cast<uint32_t>(pool->xf->pos0[i]);
    }
    return block_ids[i] * block_tokens;
}

// Source of one kind (K or V) of a block job over the job's tables, its
// items starting at `first_item`.
static BlockSource make_block_source(int type, const uint8_t *base, uint64_t block_stride,
                                     uint64_t layer_stride, const JobTables &jt, uint32_t n_layers,
                                     uint32_t block_tokens, uint32_t n_embd, uint32_t first_item,
                                     const XfParams &xp, bool is_k) {
    BlockSource s{};
    s.base = base;
    s.tables = jt.tables.dev;
    s.layer_off = is_k ? 0u : static_cast<uint32_t>(n_layers * sizeof(uint64_t));
    s.items_off = jt.items_off + 16u * first_item;
    s.theta_off = jt.theta_off;
    s.block_stride = block_stride;
    s.layer_stride = layer_stride;
    s.n_layers = n_layers;
    s.block_tokens = block_tokens;
    s.gpr = n_embd / 32;
    s.row_bytes = s.gpr * group_bytes(type);
    s.chunk_groups = chunk_groups_of(type, xp.on);
    s.chunks_per_op = (block_tokens * s.gpr + s.chunk_groups - 1) / s.chunk_groups;
    s.head_dim = xp.head_dim;
    s.n_rot = is_k ? xp.n_rot : 0u;
    s.hadamard = is_k ? xp.had_k : xp.had_v;
    s.hscale = is_k ? xp.hscale_k : xp.hscale_v;
    if (xp.lane64) {  // one workgroup per unit of 128 groups, every layer
        s.chunk_groups = kX64Groups;
        s.chunks_per_op = (block_tokens * s.gpr + kX64Groups - 1) / kX64Groups;
        s.layer_group = n_layers;
    } else {
        s.layer_group = (xp.on && s.n_rot) ? kRopeLayerGroup : 1u;
    }
    return s;
}

// One launch for K (and V when sv is set): chunks of K first, then of V.
static uint64_t block_job_chunks(const BlockSource &s, uint32_t n_items) {
    const uint64_t groups = (s.n_layers + s.layer_group - 1u) / s.layer_group;
    return static_cast<uint64_t>(n_items) * groups * s.chunks_per_op;
}

// Dynamic LDS bytes of the 64-per-lane RoPE table for chunks of `s`.
static size_t x64_tab_bytes(const BlockSource &s) {
    if (!s.n_rot) {
        return 0;
    }
    return static_cast<size_t>(chunk_rows_of(s.gpr, s.chunk_groups)) * x64_tab_geom(s.n_rot / 2).RS * 16u;
}

template <int TK>
static bool launch_x64_v(kvmem_hip_ctx *ctx, int tv, uint32_t grid, size_t tb, const BlockSource &sk,
                         const BlockSource &sv, uint32_t n_k, const ArgTables &args) {
    switch (tv) {
        case KVMEM_TYPE_Q8_0: ctx_launch(ctx, x64_kv_kernel<TK, KVMEM_TYPE_Q8_0>, dim3(grid), dim3(256), static_cast<uint32_t>(tb), sk, sv, n_k, args); break;
        case KVMEM_TYPE_Q4_0: ctx_launch(ctx, x64_kv_kernel<TK, KVMEM_TYPE_Q4_0>, dim3(grid), dim3(256), static_cast<uint32_t>(tb), sk, sv, n_k, args); break;
        case KVMEM_TYPE_Q5_0: ctx_launch(ctx, x64_kv_kernel<TK, KVMEM_TYPE_Q5_0>, dim3(grid), dim3(256), static_cast<uint32_t>(tb), sk, sv, n_k, args); break;
        case KVMEM_TYPE_F16: ctx_launch(ctx, x64_kv_kernel<TK, KVMEM_TYPE_F16>, dim3(grid), dim3(256), static_cast<uint32_t>(tb), sk, sv, n_k, args); break;
        default: fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "stage-in: unsupported V type"); return false;
    }
    return true;
}

// The job on the 64-elements-per-lane kernels (K chunks first, then V).
static bool launch_x64(kvmem_hip_ctx *ctx, int tk, int tv, uint32_t n_k, uint32_t n_v,
                       const BlockSource &sk, const BlockSource *sv, const ArgTables &args) {
    if (n_k + n_v == 0) {
        return true;
    }
    if (injected_fail(ctx, KVMEM_HIP_FAIL_LAUNCH, "stage-in transform kernel launch")) {
        return false;
    }
    const size_t tb = x64_tab_bytes(sk);  // only K is RoPE'd
    const uint32_t grid = n_k + n_v;
    bool ok = true;
    if (sv) {
        switch (tk) {
            case KVMEM_TYPE_Q8_0: ok = launch_x64_v<KVMEM_TYPE_Q8_0>(ctx, tv, grid, tb, sk, *sv, n_k, args); break;
            case KVMEM_TYPE_Q4_0: ok = launch_x64_v<KVMEM_TYPE_Q4_0>(ctx, tv, grid, tb, sk, *sv, n_k, args); break;
            case KVMEM_TYPE_Q5_0: ok = launch_x64_v<KVMEM_TYPE_Q5_0>(ctx, tv, grid, tb, sk, *sv, n_k, args); break;
            case KVMEM_TYPE_F16: ok = launch_x64_v<KVMEM_TYPE_F16>(ctx, tv, grid, tb, sk, *sv, n_k, args); break;
            default: fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "stage-in: unsupported K type"); return false;
        }
    } else {
        switch (tk) {
            case KVMEM_TYPE_Q8_0: ctx_launch(ctx, x64_kernel<KVMEM_TYPE_Q8_0>, dim3(grid), dim3(256), static_cast<uint32_t>(tb), sk, args); break;
            case KVMEM_TYPE_Q4_0: ctx_launch(ctx, x64_kernel<KVMEM_TYPE_Q4_0>, dim3(grid), dim3(256), static_cast<uint32_t>(tb), sk, args); break;
            case KVMEM_TYPE_Q5_0: ctx_launch(ctx, x64_kernel<KVMEM_TYPE_Q5_0>, dim3(grid), dim3(256), static_cast<uint32_t>(tb), sk, args); break;
            case KVMEM_TYPE_F16: ctx_launch(ctx, x64_kernel<KVMEM_TYPE_F16>, dim3(grid), dim3(256), static_cast<uint32_t>(tb), sk, args); break;
            default: fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "stage-in: unsupported K type"); return false;
        }
    }
    return ok && hip_ok(ctx, hipGetLastError(), "stage-in transform kernel launch");
}

static int launch_block_job(kvmem_hip_ctx *ctx, int type_k, const BlockSource &sk, int type_v,
                            const BlockSource *sv, uint32_t n_items, const XfParams &xp,
                            const ArgTables &args) {
    const uint64_t nk = block_job_chunks(sk, n_items);
    const uint64_t nv = sv ? block_job_chunks(*sv, n_items) : 0;
    if (nk + nv > 0x7fffffffu) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "stage-in: too many chunks in one call");
    }
    const bool xf = xp.on;
    bool ok;
    if (xp.lane64) {
        ok = launch_x64(ctx, type_k, type_v, static_cast<uint32_t>(nk), static_cast<uint32_t>(nv), sk, sv,
                        args);
    } else if (sv) {
        ok = launch_quant_kv(ctx, type_k, type_v, static_cast<uint32_t>(nk),
                             static_cast<uint32_t>(nv), sk, *sv, xf, args);
    } else {
        ok = launch_quant(ctx, type_k, static_cast<uint32_t>(nk), sk, xf, args);
    }
    return ok ? KVMEM_HIP_OK : KVMEM_HIP_ERR_RUNTIME;
}

// ---------------------------------------------------------- slot moves
//
// A set of slot moves with distinct sources and distinct destinations is a
// set of chains (s0 -> s1 -> ... -> sk) and cycles.  Chains are cut into
// segments of at most kChainSeg moves; the first source of every segment
// but a chain's first (and a cycle's first source) is saved to scratch
// beforehand, since another segment overwrites it.  One thread then carries
// one 16-byte column of a block through a whole segment with no
// synchronisation: it reads all the segment's sources, then writes all its
// destinations (straight-line code per segment length), and no other thread
// reads or writes that column of those slots.  The bytes move once, plus the saved slots, where a gather to
// scratch and a scatter back move them twice.
struct ChainParams {
    const uint8_t *tables;         // uploaded tables, or null: in the kernel's ArgTables
                                   // (K layer pointers [L], V layer pointers [L], segments)
    const uint8_t *scratch;        // entry e: [layer][T rows of K][T rows of V]
    const uint32_t *dcount;        // segment count in device memory (a device plan), or
                                   // null: one segment per grid row
    uint64_t kspan, vspan;         // one slot of one layer
    uint64_t entry_bytes;          // L * (kspan + vspan)
    uint32_t krow16, vrow16;       // row bytes / 16
    uint32_t L, T;
    uint32_t vec_per_layer;        // T * (krow16 + vrow16)
    uint32_t max_segs;             // with dcount: segments the table holds
};

// A chain segment as the kernel reads it, after the layer pointers: a
// fixed-size record of IdxT entries (16-bit when the pool's slots and
// tokens fit, else 32-bit): [len, saved + 1 (0: none), slot[0 .. 8],
// nt[0 .. 7]], padded to whole 4-byte words.  40 bytes per segment in
// 16-bit entries, so a step's table fits in the kernel arguments; one
// unconditional read of the record per workgroup.
template <typename IdxT>
constexpr uint32_t seg_record_words() {
    return (static_cast<uint32_t>(sizeof(IdxT)) * (2 * kChainSeg + 3) + 3) / 4;
}

// The N moves of one segment for one 16-byte column: N loads, then N stores
// (rows at or past a move's n_tokens are inside the slot but not stored).
// Streamed bytes: nontemporal loads and stores.
template <int N>
__device__ inline void seg_moves(const uint32_t (&slot)[kChainSeg + 1], const uint32_t (&nt)[kChainSeg],
                                 const uint8_t *first, uint8_t *base, uint64_t span, uint64_t off,
                                 uint32_t r) {
    u32x4_t val[N];
    val[0] = __builtin_nontemporal_load(as_global(reinterpret_cast<const u32x4_t *>(first)));
#pragma unroll
    for (int j = 1; j < N; ++j) {
        val[j] = __builtin_nontemporal_load(
            as_global(reinterpret_cast<const u32x4_t *>(base + static_cast<uint64_t>(slot[j]) * span + off)));
    }
#pragma unroll
    for (int j = 0; j < N; ++j) {
        if (r < nt[j]) {
            __builtin_nontemporal_store(val[j], as_global(reinterpret_cast<u32x4_t *>(
                                                    base + static_cast<uint64_t>(slot[j + 1]) * span + off)));
        }
    }
}

// grid (column blocks, segments): one 16-byte column per thread.  (Slot-
// scattered copies measured 5.9 TB/s with one column per thread and
// nontemporal accesses, 5.2 with four or eight.)  The segment's header and
// run are read once per workgroup into scalar registers.
template <typename IdxT>
__device__ inline void chain_segment(const ChainParams &p, const ArgTables &t, uint32_t seg) {
    constexpr uint32_t W = seg_record_words<IdxT>();
    const uint32_t rec = 2u * p.L * static_cast<uint32_t>(sizeof(void *)) + seg * W * 4u;
    uint32_t w[W];
#pragma unroll
    for (uint32_t i = 0; i < W; ++i) {
        w[i] = tab_read<uint32_t>(p.tables, t, rec + 4u * i);
    }
    auto entry = [&](uint32_t e) -> uint32_t {  // e is a constant after unrolling
        if constexpr (sizeof(IdxT) == 2) {
            return (w[e >> 1] >> (16u * (e & 1u))) & 0xffffu;
        } else {
            return w[e];
        }
    };
    const uint32_t len = entry(0);
    const int32_t saved = static_cast<int32_t>(entry(1)) - 1;
    uint32_t slot[kChainSeg + 1], nt[kChainSeg];
#pragma unroll
    for (uint32_t j = 0; j <= kChainSeg; ++j) {
        slot[j] = entry(2u + j);
    }
#pragma unroll
    for (uint32_t j = 0; j < kChainSeg; ++j) {
        nt[j] = entry(3u + kChainSeg + j);
    }
    const uint64_t total = static_cast<uint64_t>(p.L) * p.vec_per_layer;  // < 2^31
    const uint64_t x = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    if (x >= total) {
        return;
    }
    const uint32_t kvecs = p.T * p.krow16;
    const uint32_t l = static_cast<uint32_t>(x) / p.vec_per_layer;
    uint32_t v = static_cast<uint32_t>(x) - l * p.vec_per_layer;
    const bool is_v = v >= kvecs;
    if (is_v) {
        v -= kvecs;
    }
    const uint32_t r = v / (is_v ? p.vrow16 : p.krow16);  // row within the slot
    uint8_t *base = reinterpret_cast<uint8_t *>(
        tab_read<uint64_t>(p.tables, t, (is_v ? p.L + l : l) * static_cast<uint32_t>(sizeof(void *))));
    const uint64_t span = is_v ? p.vspan : p.kspan;
    const uint64_t off = static_cast<uint64_t>(v) * 16u;
    // Every slot of a segment is distinct (a cycle's closing source comes
    // from scratch), so all the segment's loads go first, then its stores.
    const uint8_t *first = saved >= 0
        ? p.scratch + static_cast<uint64_t>(saved) * p.entry_bytes + l * (p.kspan + p.vspan) +
              (is_v ? p.kspan : 0u) + off
        : base + static_cast<uint64_t>(slot[0]) * span + off;
    static_assert(kChainSeg == 8, "one case per segment length");
    switch (len) {  // uniform per workgroup
        case 1: seg_moves<1>(slot, nt, first, base, span, off, r); break;
        case 2: seg_moves<2>(slot, nt, first, base, span, off, r); break;
        case 3: seg_moves<3>(slot, nt, first, base, span, off, r); break;
        case 4: seg_moves<4>(slot, nt, first, base, span, off, r); break;
        case 5: seg_moves<5>(slot, nt, first, base, span, off, r); break;
        case 6: seg_moves<6>(slot, nt, first, base, span, off, r); break;
        case 7: seg_moves<7>(slot, nt, first, base, span, off, r); break;
        case 8: seg_moves<8>(slot, nt, first, base, span, off, r); break;
        default: break;
    }
}

template <typename IdxT>
__global__ __launch_bounds__(256) void move_chain_kernel(ChainParams p, ArgTables t) {
    if (p.dcount) {  // a device plan: the grid's rows take the segments in turn
        const uint32_t n = min(*p.dcount, p.max_segs);
        for (uint32_t seg = blockIdx.y; seg < n; seg += gridDim.y) {
            chain_segment<IdxT>(p, t, seg);
        }
        return;
    }
    chain_segment<IdxT>(p, t, blockIdx.y);
}

// The kernel's table for `segs`: layer pointers, then one record per segment.
template <typename IdxT>
static void chain_table(const kvmem_hip_pool *pool, bool want_v, const std::vector<ChainSeg> &segs,
                        std::vector<uint8_t> &table) {
    const uint32_t L = pool->n_layers;
    const size_t ptr_bytes = 2 * L * sizeof(void *);
    const size_t rec_bytes = 4 * seg_record_words<IdxT>();
    table.assign(ptr_bytes + segs.size() * rec_bytes, 0);
    std::memcpy(table.data(), pool->k_layers, L * sizeof(void *));
    if (want_v) {
        std::memcpy(table.data() + L * sizeof(void *), pool->v_layers, L * sizeof(void *));
    }
    for (size_t i = 0; i < segs.size(); ++i) {
        const ChainSeg &sg = segs[i];
        IdxT *r = reinterpret_cast<IdxT *>(table.data() + ptr_bytes + i * rec_bytes);
        r[0] = static_cast<IdxT>(sg.len);
        r[1] = static_cast<IdxT>(sg.saved + 1);
        for (int j = 0; j <= kChainSeg; ++j) {
            r[2 + j] = static_cast<IdxT>(sg.slot[j]);
        }
        for (int j = 0; j < kChainSeg; ++j) {
            r[3 + kChainSeg + j] = static_cast<IdxT>(sg.nt[j]);
        }
    }
}

// ------------------------------------------------ device reselect plan
//
// apply_retrieval as one device pipeline: the top-k kernel leaves the
// selection in device memory, and plan_kernel (one workgroup) diffs it
// against the pool's resident blocks and writes the job tables of the
// kernels queued behind it: the stage-in items, the chain segments of the
// slot moves and the copies that save cut slots first.  Window slot i takes
// the i-th selected block (canonical layout).  A selected block resident at
// slot s moves s -> i when s != i, unless it is the grown partial tail,
// which is staged again; a selected block not resident is staged into slot
// i.  Moves then have distinct sources and distinct destinations.  With the
// resident blocks at slots ascending with their ids (a canonical pool)
// sources and destinations both ascend with the block id, so the moves
// form chains and never a cycle.
//
// A chain starts at a move whose source no move writes; pred(m) is the move
// that writes m's source, which m must read first (inside a segment the walk
// reads every source before it writes; across segments the cut slot is
// read from its saved copy).  Each move's rank along its chain comes from pointer jumping on pred
// (11 rounds cover kPlanMaxSel moves).  Segments of kChainSeg moves start at
// ranks 0, kChainSeg, ...; the first source of every segment but a chain's
// first is saved to scratch beforehand, as build_chains (move_plan.cpp)
// does on the host.
constexpr uint32_t kPlanThreads = 1024;
constexpr uint32_t kChainRows = 64;  // chain segments the device plan's walk runs side by side
constexpr uint32_t kPlanMaxSel = KVMEM_PLAN_MAX_SEL;    // selected blocks per step (one per thread)
constexpr uint32_t kPlanMaxSlots = KVMEM_PLAN_MAX_SLOTS;  // pool slots
constexpr uint16_t kNoMove = 0xffffu;
constexpr uint32_t kPlanJumpRounds = 11;  // 2^11 > kPlanMaxSel
constexpr uint32_t kPlanSaveOpsPer(uint32_t L) { return 2u * L; }
static_assert(kChainSeg == 8, "plan segments are the chain kernel's");

// Counts at the start of the plan buffer (and in host-mapped memory).
enum PlanCount : uint32_t {
    kPlanStage = 0,   // blocks staged
    kPlanMoves = 1,   // slot moves
    kPlanSegs = 2,    // chain segments
    kPlanSaves = 3,   // slots saved before the walk
    kPlanSaveOps = 4, // their copies (K and V of every layer)
    kPlanSel = 5,     // selected blocks
    kPlanError = 6,   // nonzero: the plan was refused (nothing moves)
    kPlanRows = 7,    // rows the moves carry (sum over moves of n_tokens)
    kPlanCounts = 16
};

struct PlanParams {
    const uint32_t *sel;     // [0] = selected count, then the ascending ids
    uint8_t *plan;           // counts, stage table, chain table, save copies
    uint32_t *counts_host;   // the counts again, host-mapped
    const uint8_t *scratch;  // saved slot e at scratch + e * entry_bytes
    const uint8_t *tables;   // uploaded pool/resident table, or null: in the ArgTables
    uint64_t kspan, vspan;   // one slot of one layer
    uint64_t entry_bytes;    // L * (kspan + vspan)
    uint32_t off_stage, off_chain, off_saves;
    uint32_t n_res, n_slots, n_blocks, T, last_T, dirty, L, max_sel, max_saves;
    uint32_t first_T;        // tokens of block 0
    uint32_t n_theta;        // RoPE frequencies copied from the tables to the stage table
    uint32_t theta_src;      // their byte offset in the tables
    uint32_t theta_dst;      // and in the stage table
};

// Exclusive prefix over the workgroup's threads of `v`; `total` gets the sum.
__device__ inline uint32_t plan_scan(uint32_t v, uint32_t *wave_tot, uint32_t &total) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    constexpr uint32_t kWaves = kPlanThreads / 64u;
    uint32_t x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(x, off, 64);
        if (lane >= static_cast<uint32_t>(off)) {
            x += y;
        }
    }
    if (lane == 63u) {
        wave_tot[wave] = x;
    }
    __syncthreads();
    uint32_t before = 0;
    total = 0;
    for (uint32_t w = 0; w < kWaves; ++w) {
        const uint32_t tw = wave_tot[w];
        before += w < wave ? tw : 0u;
        total += tw;
    }
    __syncthreads();  // wave_tot is rewritten by the next scan
    return before + x - v;
}

__global__ __launch_bounds__(kPlanThreads) void plan_kernel(PlanParams p, ArgTables t) {
    __shared__ uint32_t res_block[kPlanMaxSlots];
    __shared__ uint16_t res_slot[kPlanMaxSlots];
    __shared__ uint16_t at_src[kPlanMaxSlots];  // move reading slot s
    __shared__ uint16_t at_dst[kPlanMaxSlots];  // move writing slot s
    __shared__ uint16_t msrc[kPlanMaxSel], mdst[kPlanMaxSel], mnt[kPlanMaxSel], mnext[kPlanMaxSel];
    __shared__ uint16_t jump[kPlanMaxSel];
    __shared__ uint32_t rank[kPlanMaxSel];
    __shared__ uint32_t wave_tot[kPlanThreads / 64u];
    __shared__ uint32_t s_bad;
    const uint32_t tid = threadIdx.x;
    const uint32_t L = p.L;
    // the pool's layer pointers head the stage and chain tables
    for (uint32_t j = tid; j < 2u * L; j += kPlanThreads) {
        const uint64_t v = tab_read<uint64_t>(p.tables, t, 8u * j);
        *reinterpret_cast<uint64_t *>(p.plan + p.off_stage + 8u * j) = v;
        *reinterpret_cast<uint64_t *>(p.plan + p.off_chain + 8u * j) = v;
    }
    // the RoPE frequencies of a transformed stage-in follow its items
    for (uint32_t j = tid; j < p.n_theta; j += kPlanThreads) {
        *reinterpret_cast<float *>(p.plan + p.off_stage + p.theta_dst + 4u * j) =
            tab_read<float>(p.tables, t, p.theta_src + 4u * j);
    }
    const uint32_t rb_off = 16u * L;
    const uint32_t rs_off = rb_off + 4u * p.n_res;
    for (uint32_t r = tid; r < p.n_res; r += kPlanThreads) {
        res_block[r] = tab_read<uint32_t>(p.tables, t, rb_off + 4u * r);
        res_slot[r] = static_cast<uint16_t>(tab_read<uint32_t>(p.tables, t, rs_off + 4u * r));
    }
    for (uint32_t q = tid; q < p.n_slots; q += kPlanThreads) {
        at_src[q] = kNoMove;
        at_dst[q] = kNoMove;
    }
    if (tid == 0) {
        s_bad = 0;
    }
    __syncthreads();

    // ---- selected index i = tid: stays, moves or is staged
    const uint32_t k = min(p.sel[0], p.max_sel);
    const uint32_t i = tid;
    uint32_t b = 0;
    int32_t src = -1;
    if (i < k) {
        b = p.sel[1u + i];
        uint32_t lo = 0, hi = p.n_res;  // first resident id >= b
        while (lo < hi) {
            const uint32_t mid = (lo + hi) >> 1;
            if (res_block[mid] < b) {
                lo = mid + 1u;
            } else {
                hi = mid;
            }
        }
        if (lo < p.n_res && res_block[lo] == b && b != p.dirty) {
            src = res_slot[lo];
        }
        if (b >= p.n_blocks) {
            atomicOr(&s_bad, 1u);
        }
    }
    const bool stage = i < k && src < 0;
    const bool move = i < k && src >= 0 && static_cast<uint32_t>(src) != i;
    const uint32_t nt = (b + 1u == p.n_blocks && p.last_T != 0u) ? p.last_T : p.T;
    uint32_t n_stage, n_moves;
    const uint32_t at_stage = plan_scan(stage ? 1u : 0u, wave_tot, n_stage);
    const uint32_t m_own = plan_scan(move ? 1u : 0u, wave_tot, n_moves);
    if (stage) {
        uint32_t *item = reinterpret_cast<uint32_t *>(p.plan + p.off_stage + 16u * L + 16u * at_stage);
        const bool ok = b < p.n_blocks;
        item[0] = ok ? b : 0u;
        item[1] = i;
        item[2] = ok ? nt : p.first_T;
        item[3] = ok ? b * p.T : 0u;
    }
    // the host launches the stage-in with its own count, at most max_sel:
    // every entry up to there holds an in-bounds item (block 0 to slot 0),
    // whatever the two plans make of the selection; a disagreement is
    // caught afterwards and drops the window
    if (tid >= n_stage && tid < p.max_sel) {
        uint32_t *item = reinterpret_cast<uint32_t *>(p.plan + p.off_stage + 16u * L + 16u * tid);
        item[0] = 0u;
        item[1] = 0u;
        item[2] = p.first_T;
        item[3] = 0u;
    }
    if (move) {
        msrc[m_own] = static_cast<uint16_t>(src);
        mdst[m_own] = static_cast<uint16_t>(i);
        mnt[m_own] = static_cast<uint16_t>(nt);
        at_src[src] = static_cast<uint16_t>(m_own);
        at_dst[i] = static_cast<uint16_t>(m_own);
    }
    __syncthreads();

    // ---- chains: rank of move m = tid along its chain
    const uint32_t m = tid;
    uint16_t jm = kNoMove;
    uint32_t rm = 0;
    if (m < n_moves) {
        jm = at_dst[msrc[m]];             // pred: the move writing m's source
        mnext[m] = at_src[mdst[m]];       // next: the move reading m's destination
        rm = jm != kNoMove ? 1u : 0u;
        jump[m] = jm;
        rank[m] = rm;
    }
    __syncthreads();
    for (uint32_t round = 0; round < kPlanJumpRounds; ++round) {
        uint16_t j2 = kNoMove;
        uint32_t r2 = 0;
        if (m < n_moves && jm != kNoMove) {
            j2 = jump[jm];
            r2 = rank[jm];
        }
        __syncthreads();
        if (m < n_moves && jm != kNoMove) {
            rm += r2;
            jm = j2;
            jump[m] = jm;
            rank[m] = rm;
        }
        __syncthreads();
    }
    if (m < n_moves && jm != kNoMove) {
        atomicOr(&s_bad, 2u);  // a cycle: this plan is refused
    }

    // ---- segments from ranks 0, kChainSeg, ...; the non-first ones save
    const bool seg_start = m < n_moves && (rm % kChainSeg) == 0u;
    const bool saves = seg_start && rm > 0u;
    uint32_t n_segs, n_saves;
    const uint32_t g = plan_scan(seg_start ? 1u : 0u, wave_tot, n_segs);
    const uint32_t e = plan_scan(saves ? 1u : 0u, wave_tot, n_saves);
    uint32_t rows = 0, n_rows = 0;
    if (m < n_moves) {
        rows = mnt[m];
    }
    (void) plan_scan(rows, wave_tot, n_rows);
    if (seg_start) {
        // the record [len, saved + 1, slot[0 .. 8], nt[0 .. 7]] of 16-bit
        // entries, padded to whole words; every index is a constant after
        // unrolling, so the entries stay in registers
        uint32_t rec[2 * kChainSeg + 4];
#pragma unroll
        for (uint32_t q = 0; q < 2 * kChainSeg + 4; ++q) {
            rec[q] = 0u;
        }
        uint32_t len = 0;
        uint32_t j = m;
        rec[2] = msrc[m];
#pragma unroll
        for (uint32_t q = 0; q < kChainSeg; ++q) {
            if (j != kNoMove) {
                rec[3 + q] = mdst[j];
                rec[3 + kChainSeg + q] = mnt[j];
                len = q + 1u;
                j = mnext[j];
            }
        }
        rec[0] = len;
        rec[1] = saves ? e + 1u : 0u;
        constexpr uint32_t W = seg_record_words<uint16_t>();
        static_assert(2 * W <= 2 * kChainSeg + 4, "record entries");
        uint32_t *dst = reinterpret_cast<uint32_t *>(p.plan + p.off_chain + 16u * L + 4u * W * g);
#pragma unroll
        for (uint32_t w = 0; w < W; ++w) {
            dst[w] = (rec[2 * w] & 0xffffu) | (rec[2 * w + 1] << 16);
        }
        if (saves && e < p.max_saves) {
            CopyOpDev *ops = reinterpret_cast<CopyOpDev *>(p.plan + p.off_saves) + kPlanSaveOpsPer(L) * e;
            const uint8_t *entry = p.scratch + e * p.entry_bytes;
            for (uint32_t l = 0; l < L; ++l) {
                const uint8_t *kl = reinterpret_cast<const uint8_t *>(tab_read<uint64_t>(p.tables, t, 8u * l));
                const uint8_t *vl = reinterpret_cast<const uint8_t *>(tab_read<uint64_t>(p.tables, t, 8u * (L + l)));
                uint8_t *at = const_cast<uint8_t *>(entry) + l * (p.kspan + p.vspan);
                ops[2 * l] = CopyOpDev{kl + msrc[m] * p.kspan, at, p.kspan};
                ops[2 * l + 1] = CopyOpDev{vl + msrc[m] * p.vspan, at + p.kspan, p.vspan};
            }
        }
    }
    __syncthreads();
    if (tid == 0) {
        const uint32_t bad = s_bad | (n_saves > p.max_saves ? 4u : 0u);
        uint32_t c[kPlanCounts] = {};
        c[kPlanStage] = bad ? 0u : n_stage;
        c[kPlanMoves] = n_moves;
        c[kPlanSegs] = bad ? 0u : n_segs;
        c[kPlanSaves] = n_saves;
        c[kPlanSaveOps] = bad ? 0u : n_saves * kPlanSaveOpsPer(L);
        c[kPlanSel] = k;
        c[kPlanError] = bad;
        c[kPlanRows] = n_rows;
        uint32_t *dc = reinterpret_cast<uint32_t *>(p.plan);
        for (uint32_t q = 0; q < kPlanCounts; ++q) {
            dc[q] = c[q];
            p.counts_host[q] = c[q];
        }
    }
}

bool load_stagein_kernels() {
    return load_kernel_object(&quant_scatter_kv_kernel<KVMEM_TYPE_Q8_0, KVMEM_TYPE_Q8_0, false, false>);
}

}  // namespace kvmem_hip

using namespace kvmem_hip;

extern "C" {

int kvmem_hip_stagein_quant(kvmem_hip_ctx *ctx, const kvmem_hip_quant_op *ops, int n_ops) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (n_ops <= 0) {
        return KVMEM_HIP_OK;
    }
    if (!ops) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "stagein_quant: null ops");
    }
    (void) hipSetDevice(ctx->device);
    const int types[4] = {KVMEM_TYPE_Q8_0, KVMEM_TYPE_Q5_0, KVMEM_TYPE_Q4_0, KVMEM_TYPE_F16};
    for (int i = 0; i < n_ops; ++i) {
        const kvmem_hip_quant_op &op = ops[i];
        if (!kvmem_hip_quant_ok(op.type)) {
            return fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "stagein_quant: unsupported type");
        }
        const uint32_t stride = op.src_stride ? op.src_stride : op.n_embd * 2u;
        if (op.n_rows == 0) {
            continue;
        }
        if (!op.src || !op.dst || op.n_embd == 0 || op.n_embd % 32 != 0 || !aligned16(op.src) ||
            !aligned16(op.dst) || stride % 16 != 0 || stride < op.n_embd * 2u) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID,
                        "stagein_quant: op needs 16-byte aligned src/dst/stride and n_embd % 32 == 0");
        }
    }
    PerfScope timed(ctx, kPerfSet);
    for (int type : types) {
        std::vector<QuantOpDev> dev;
        uint64_t chunks = 0;
        const uint32_t cg = chunk_groups_of(type, false);
        for (int i = 0; i < n_ops; ++i) {
            const kvmem_hip_quant_op &op = ops[i];
            if (op.type != type || op.n_rows == 0) {
                continue;
            }
            QuantOpDev d;
            d.src = static_cast<const uint8_t *>(op.src);
            d.dst = static_cast<uint8_t *>(op.dst);
            d.gpr = op.n_embd / 32;
            d.n_groups = op.n_rows * d.gpr;
            d.src_stride = op.src_stride ? op.src_stride : op.n_embd * 2u;
            d.chunk0 = static_cast<uint32_t>(chunks);
            chunks += (d.n_groups + cg - 1) / cg;
            dev.push_back(d);
        }
        if (dev.empty()) {
            continue;
        }
        if (chunks > 0x7fffffffu) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID, "stagein_quant: too many chunks");
        }
        void *ops_dev = upload(ctx, dev.data(), dev.size() * sizeof(QuantOpDev), "stagein_quant ops");
        if (!ops_dev) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        OpListSource s{static_cast<const QuantOpDev *>(ops_dev), static_cast<uint32_t>(dev.size()), cg};
        if (!launch_quant(ctx, type, static_cast<uint32_t>(chunks), s)) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
    }
    timed.ok();
    return KVMEM_HIP_OK;
}

int kvmem_hip_stagein_blocks(kvmem_hip_ctx *ctx, const kvmem_hip_history *hist,
                             const kvmem_hip_pool *pool, const uint32_t *block_ids,
                             const uint32_t *slots, uint32_t n) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (n == 0) {
        return KVMEM_HIP_OK;
    }
    if (!hist || !hist->k || !block_ids || !slots) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "stagein_blocks: null argument");
    }
    const bool want_v = hist->v != nullptr && pool && pool->v_layers != nullptr;
    const uint32_t T = hist->block_tokens;
    if (T == 0 || hist->n_embd_k % 32 != 0 || (want_v && hist->n_embd_v % 32 != 0) ||
        !aligned16(hist->k) || (want_v && !aligned16(hist->v))) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "stagein_blocks: bad history geometry/alignment");
    }
    const uint32_t cap = hist->capacity_blocks ? hist->capacity_blocks : hist->n_blocks;
    if (cap < hist->n_blocks) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "stagein_blocks: capacity_blocks below n_blocks");
    }
    int st = check_pool(ctx, pool, hist->n_layers, T, hist->n_embd_k, hist->n_embd_v, want_v);
    if (st != KVMEM_HIP_OK) {
        return st;
    }
    XfParams xp;
    st = resolve_xf(ctx, pool, hist->n_embd_k, hist->n_embd_v, want_v, xp);
    if (st != KVMEM_HIP_OK) {
        return st;
    }
    std::vector<uint32_t> items(4 * static_cast<size_t>(n));
    for (uint32_t i = 0; i < n; ++i) {
        if (block_ids[i] >= hist->n_blocks || slots[i] >= pool->n_slots) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID, "stagein_blocks: block id or slot out of range");
        }
        const bool last = block_ids[i] + 1 == hist->n_blocks && hist->last_block_tokens != 0;
        items[4 * i + 0] = block_ids[i];
        items[4 * i + 1] = slots[i];
        items[4 * i + 2] = last ? std::min(hist->last_block_tokens, T) : T;
        items[4 * i + 3] = item_pos0(pool, block_ids, i, T);
    }
    (void) hipSetDevice(ctx->device);
    JobTables jt;
    if (!stage_block_job(ctx, pool, want_v, items, xp, jt)) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    const uint64_t bk = static_cast<uint64_t>(T) * hist->n_embd_k * 2u;
    const BlockSource sk = make_block_source(pool->type_k, static_cast<const uint8_t *>(hist->k), bk,
                                             bk * cap, jt, hist->n_layers, T,
                                             hist->n_embd_k, 0, xp, true);
    BlockSource sv{};
    if (want_v) {
        const uint64_t bv = static_cast<uint64_t>(T) * hist->n_embd_v * 2u;
        sv = make_block_source(pool->type_v, static_cast<const uint8_t *>(hist->v), bv,
                               bv * cap, jt, hist->n_layers, T,
                               hist->n_embd_v, 0, xp, false);
    }
    PerfLaunchScope timed(ctx, kPerfSet);  // one launch: the events ride on it
    st = launch_block_job(ctx, pool->type_k, sk, pool->type_v, want_v ? &sv : nullptr, n, xp, jt.tables.args);
    if (st == KVMEM_HIP_OK) {
        timed.ok();
    }
    return st;
}

int kvmem_hip_stagein_blocks_host(kvmem_hip_ctx *ctx, const kvmem_hip_host_history *hist,
                                  const kvmem_hip_pool *pool, const uint32_t *block_ids,
                                  const uint32_t *slots, uint32_t n) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (n == 0) {
        return KVMEM_HIP_OK;
    }
    if (!hist || !hist->base || !block_ids || !slots || !pool) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "stagein_blocks_host: null argument");
    }
    const uint32_t T = hist->block_tokens;
    const uint32_t L = hist->n_layers;
    const bool want_v = hist->n_embd_v != 0 && pool->v_layers != nullptr;
    if (T == 0 || hist->n_embd_k % 32 != 0 || hist->n_embd_v % 32 != 0) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "stagein_blocks_host: bad geometry");
    }
    int st = check_pool(ctx, pool, L, T, hist->n_embd_k, hist->n_embd_v, want_v);
    if (st != KVMEM_HIP_OK) {
        return st;
    }
    const uint64_t kbytes = static_cast<uint64_t>(T) * hist->n_embd_k * 2u;
    const uint64_t vbytes = static_cast<uint64_t>(T) * hist->n_embd_v * 2u;
    const uint64_t layer_bytes = kbytes + vbytes;
    const uint64_t span = layer_bytes * L;  // one block, every layer, K then V
    for (uint32_t i = 0; i < n; ++i) {
        if (block_ids[i] >= hist->n_blocks || slots[i] >= pool->n_slots) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID, "stagein_blocks_host: block id or slot out of range");
        }
    }
    XfParams xp;
    st = resolve_xf(ctx, pool, hist->n_embd_k, hist->n_embd_v, want_v, xp);
    if (st != KVMEM_HIP_OK) {
        return st;
    }
    (void) hipSetDevice(ctx->device);
    // Pinned history: the kernel reads the blocks over the link itself, one
    // launch for every block, no ring and no copy calls (the copies cost the
    // link ~10 us each between them).
    if (const uint8_t *view = host_device_view(hist->base, span * hist->n_blocks)) {
        std::vector<uint32_t> items(4 * static_cast<size_t>(n));
        for (uint32_t i = 0; i < n; ++i) {
            const uint32_t b = block_ids[i];
            items[4 * i + 0] = b;
            items[4 * i + 1] = slots[i];
            items[4 * i + 2] = (b + 1 == hist->n_blocks && hist->last_block_tokens != 0)
                                   ? std::min(hist->last_block_tokens, T) : T;
            items[4 * i + 3] = item_pos0(pool, block_ids, i, T);
        }
        JobTables jt;
        if (!stage_block_job(ctx, pool, want_v, items, xp, jt)) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        const BlockSource sk = make_block_source(pool->type_k, view, span, layer_bytes, jt, L, T,
                                                 hist->n_embd_k, 0, xp, true);
        BlockSource sv{};
        if (want_v) {
            sv = make_block_source(pool->type_v, view + kbytes, span, layer_bytes, jt, L, T,
                                   hist->n_embd_v, 0, xp, false);
        }
        PerfLaunchScope timed(ctx, kPerfSet);  // one launch: the events ride on it
        st = launch_block_job(ctx, pool->type_k, sk, pool->type_v, want_v ? &sv : nullptr, n, xp, jt.tables.args);
        if (st == KVMEM_HIP_OK) {
            timed.ok();
            // the kernel reads each block's rows of every layer over the link
            uint64_t rows = 0;
            for (uint32_t i = 0; i < n; ++i) rows += items[4 * i + 2];
            note_xfer(ctx, kXferH2D, rows * L * (want_v ? kbytes + vbytes : kbytes) / T);
        }
        return st;
    }
    // Pageable history: device ring of kH2dRing slots of 32 MiB or more (at
    // least one block each), filled by runtime copies.
    if (!ensure_h2d_ring(ctx, span)) {
        return KVMEM_HIP_ERR_NOMEM;  // the failing call is in kvmem_hip_last_error
    }
    constexpr int kRing = kH2dRing;
    const uint64_t slot_bytes = ctx->h2d_slot_bytes;
    const uint32_t per_slot = static_cast<uint32_t>(slot_bytes / span);
    // items of every batch, block index relative to its ring slot
    std::vector<uint32_t> items(4 * static_cast<size_t>(n));
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t b = block_ids[i];
        items[4 * i + 0] = i % per_slot;
        items[4 * i + 1] = slots[i];
        items[4 * i + 2] = (b + 1 == hist->n_blocks && hist->last_block_tokens != 0)
                               ? std::min(hist->last_block_tokens, T) : T;
        items[4 * i + 3] = item_pos0(pool, block_ids, i, T);
    }
    JobTables jt;
    if (!stage_block_job(ctx, pool, want_v, items, xp, jt)) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    PerfScope timed(ctx, kPerfSet);
    const uint8_t *host = static_cast<const uint8_t *>(hist->base);
    uint8_t *ring = static_cast<uint8_t *>(ctx->h2d_ring.ptr);
    int r = 0;
    for (uint32_t first = 0; first < n; first += per_slot) {
        const uint32_t cnt = std::min(per_slot, n - first);
        uint8_t *slot_base = ring + static_cast<uint64_t>(r) * slot_bytes;
        // the previous kernel reading this ring slot must be done
        if (!hip_ok(ctx, hipStreamWaitEvent(ctx->copy_stream, ctx->h2d_consumed[r], 0), "h2d wait consumed")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        for (uint32_t j = 0; j < cnt; ++j) {
            // a run of consecutive blocks comes in as one copy
            const uint32_t b = block_ids[first + j];
            uint32_t run = 1;
            while (j + run < cnt && block_ids[first + j + run] == b + run) {
                ++run;
            }
            if (injected_fail(ctx, KVMEM_HIP_FAIL_COPY, "h2d block copy")) {
                return KVMEM_HIP_ERR_RUNTIME;
            }
            if (!hip_ok(ctx, hipMemcpyAsync(slot_base + j * span, host + static_cast<uint64_t>(b) * span,
                                            run * span, hipMemcpyHostToDevice, ctx->copy_stream),
                        "h2d block copy")) {
                return KVMEM_HIP_ERR_RUNTIME;
            }
            note_xfer(ctx, kXferH2D, run * span);
            j += run - 1;
        }
        if (!hip_ok(ctx, hipEventRecord(ctx->h2d_copied[r], ctx->copy_stream), "h2d record") ||
            !hip_ok(ctx, hipStreamWaitEvent(ctx->stream, ctx->h2d_copied[r], 0), "h2d wait copied")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        const BlockSource sk = make_block_source(pool->type_k, slot_base, span, layer_bytes, jt,
                                                 L, T, hist->n_embd_k, first, xp, true);
        BlockSource sv{};
        if (want_v) {
            sv = make_block_source(pool->type_v, slot_base + kbytes, span, layer_bytes, jt, L,
                                   T, hist->n_embd_v, first, xp, false);
        }
        st = launch_block_job(ctx, pool->type_k, sk, pool->type_v, want_v ? &sv : nullptr, cnt, xp, jt.tables.args);
        if (st != KVMEM_HIP_OK) {
            return st;
        }
        if (!hip_ok(ctx, hipEventRecord(ctx->h2d_consumed[r], ctx->stream), "h2d record consumed")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        r = (r + 1) % kRing;
    }
    timed.ok();
    return KVMEM_HIP_OK;
}

int kvmem_hip_move_slots(kvmem_hip_ctx *ctx, const kvmem_hip_pool *pool, const uint32_t *src_slots,
                         const uint32_t *dst_slots, const uint32_t *n_tokens, uint32_t n) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (n == 0) {
        return KVMEM_HIP_OK;
    }
    if (!pool || !pool->k_layers || !src_slots || !dst_slots) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "move_slots: null argument");
    }
    const bool want_v = pool->v_layers != nullptr;
    const uint64_t krow = kvmem_hip_row_size(pool->type_k, pool->n_embd_k);
    const uint64_t vrow = want_v ? kvmem_hip_row_size(pool->type_v, pool->n_embd_v) : 0;
    const uint64_t kspan = krow * pool->block_tokens;
    const uint64_t vspan = vrow * pool->block_tokens;
    if (kspan == 0 || (want_v && vspan == 0)) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "move_slots: bad pool geometry");
    }
    for (uint32_t i = 0; i < n; ++i) {
        if (src_slots[i] >= pool->n_slots || dst_slots[i] >= pool->n_slots) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID, "move_slots: slot out of range");
        }
        if (n_tokens && n_tokens[i] > pool->block_tokens) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID, "move_slots: n_tokens above block_tokens");
        }
    }
    // every layer tensor the moves touch; the chain walk's 16-byte accesses
    // also need them 16-byte aligned (else the moves gather and scatter)
    bool aligned = true;
    for (uint32_t l = 0; l < pool->n_layers; ++l) {
        if (!pool->k_layers[l] || (want_v && !pool->v_layers[l])) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID, "move_slots: null layer tensor");
        }
        aligned = aligned && aligned16(pool->k_layers[l]) && (!want_v || aligned16(pool->v_layers[l]));
    }
    const uint64_t per_move = (kspan + vspan) * pool->n_layers;
    (void) hipSetDevice(ctx->device);
    // distinct sources and destinations, 16-byte rows: chains, bytes moved once
    std::vector<ChainSeg> segs;
    std::vector<uint32_t> saved;
    if (aligned && krow % 16 == 0 && vrow % 16 == 0 &&
        build_chains(src_slots, dst_slots, n_tokens, n, pool->block_tokens, pool->n_slots, segs, saved) &&
        segs.size() <= 65535) {
        if (segs.empty()) {
            return KVMEM_HIP_OK;
        }
        if (!saved.empty() && !ensure_dev(ctx, ctx->move_scratch, per_move * saved.size(), "move_slots scratch")) {
            return KVMEM_HIP_ERR_NOMEM;
        }
        uint8_t *scratch = static_cast<uint8_t *>(ctx->move_scratch.ptr);
        std::vector<CopyOpDev> ops;
        for (size_t e = 0; e < saved.size(); ++e) {
            uint8_t *sc = scratch + per_move * e;
            for (uint32_t l = 0; l < pool->n_layers; ++l) {
                ops.push_back({static_cast<const uint8_t *>(pool->k_layers[l]) + saved[e] * kspan, sc, kspan});
                sc += kspan;
                if (want_v) {
                    ops.push_back({static_cast<const uint8_t *>(pool->v_layers[l]) + saved[e] * vspan, sc, vspan});
                    sc += vspan;
                }
            }
        }
        // the K and V layer tables, then the segments (in the kernel arguments when they fit)
        const uint32_t L = pool->n_layers;
        // 16-bit records when every slot, row count and saved entry fits
        const bool narrow = pool->n_slots <= 65536u && pool->block_tokens <= 65535u && saved.size() < 65535u;
        std::vector<uint8_t> table;
        if (narrow) {
            chain_table<uint16_t>(pool, want_v, segs, table);
        } else {
            chain_table<uint32_t>(pool, want_v, segs, table);
        }
        LaunchTables chain_tables;
        if (!stage_tables(ctx, table.data(), table.size(), chain_tables, "move_slots chains")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        uint64_t moved = 0;
        for (const ChainSeg &sg : segs) {
            for (uint32_t j = 0; j < sg.len; ++j) {
                moved += static_cast<uint64_t>(sg.nt[j]) * (krow + vrow) * L;
            }
        }
        ChainParams cp{};
        cp.tables = chain_tables.dev;
        cp.scratch = scratch;
        cp.kspan = kspan;
        cp.vspan = vspan;
        cp.entry_bytes = per_move;
        cp.krow16 = static_cast<uint32_t>(krow / 16);
        cp.vrow16 = static_cast<uint32_t>(vrow / 16);
        cp.L = L;
        cp.T = pool->block_tokens;
        cp.vec_per_layer = cp.T * (cp.krow16 + cp.vrow16);
        const uint64_t nvec = static_cast<uint64_t>(L) * cp.vec_per_layer;
        if (nvec > 0x7fffffffu) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID, "move_slots: slot too large");
        }
        LaunchTables save_tables;
        if (!ops.empty() && !stage_copy_ops(ctx, ops, save_tables, "move_slots save")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        PerfScope timed(ctx, kPerfLayout);
        if (!launch_staged_copies(ctx, save_tables, ops.size(), max_op_bytes(ops), "move_slots save")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        if (!ops.empty()) {
            note_xfer(ctx, kXferD2D, per_move * saved.size());
        }
        const dim3 grid(static_cast<uint32_t>((nvec + 255) / 256), static_cast<uint32_t>(segs.size()));
        if (injected_fail(ctx, KVMEM_HIP_FAIL_LAUNCH, "move_slots chain launch")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        if (narrow) {
            move_chain_kernel<uint16_t><<<grid, 256, 0, ctx->stream>>>(cp, chain_tables.args);
        } else {
            move_chain_kernel<uint32_t><<<grid, 256, 0, ctx->stream>>>(cp, chain_tables.args);
        }
        if (!hip_ok(ctx, hipGetLastError(), "move_slots chain launch")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        timed.ok();
        note_xfer(ctx, kXferD2D, moved);
        return KVMEM_HIP_OK;
    }
    if (!ensure_dev(ctx, ctx->move_scratch, per_move * n, "move_slots scratch")) {
        return KVMEM_HIP_ERR_NOMEM;
    }
    uint8_t *scratch = static_cast<uint8_t *>(ctx->move_scratch.ptr);
    std::vector<const void *> gs, ss;
    std::vector<void *> gd, sd;
    std::vector<size_t> nb;
    for (uint32_t i = 0; i < n; ++i) {
        const uint64_t nt = n_tokens ? n_tokens[i] : pool->block_tokens;
        if (nt == 0) {
            continue;  // nothing of this block to move
        }
        uint8_t *sc = scratch + per_move * i;
        for (uint32_t l = 0; l < pool->n_layers; ++l) {
            uint8_t *kb = static_cast<uint8_t *>(pool->k_layers[l]);
            gs.push_back(kb + src_slots[i] * kspan);
            gd.push_back(sc);
            ss.push_back(sc);
            sd.push_back(kb + dst_slots[i] * kspan);
            nb.push_back(nt * krow);
            sc += kspan;
            if (want_v) {
                uint8_t *vb = static_cast<uint8_t *>(pool->v_layers[l]);
                gs.push_back(vb + src_slots[i] * vspan);
                gd.push_back(sc);
                ss.push_back(sc);
                sd.push_back(vb + dst_slots[i] * vspan);
                nb.push_back(nt * vrow);
                sc += vspan;
            }
        }
    }
    if (nb.empty()) {
        return KVMEM_HIP_OK;
    }
    const int nops = static_cast<int>(nb.size());
    int st = kvmem_hip_d2d_batched(ctx, gs.data(), gd.data(), nb.data(), nops);
    if (st == KVMEM_HIP_OK) {
        st = kvmem_hip_d2d_batched(ctx, ss.data(), sd.data(), nb.data(), nops);
    }
    return st;
}


// Internal to the library (the reselect engine's device pipeline): the plan
// kernel over the selection the last topk_launch(to_device) leaves in
// ctx->topk_dev, then the slot saves, the chain walk and the stage-in, all
// sized on the device.  res_block / res_slot: the blocks whose pool rows are
// valid, ascending in id and in slot; dirty: a resident block to stage again
// (UINT32_MAX: none); max_sel: the largest selection the top-k can return.
int kvmem_hip_reselect_device(kvmem_hip_ctx *ctx, const kvmem_hip_history *hist, const kvmem_hip_pool *pool,
                              const uint32_t *res_block, const uint32_t *res_slot, uint32_t n_res,
                              uint32_t dirty, uint32_t max_sel) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (!hist || !hist->k || !hist->v || !pool || !pool->v_layers || (n_res && (!res_block || !res_slot))) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "reselect_device: null argument");
    }
    if (!ctx->topk_pending || !ctx->topk_dev.ptr) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "reselect_device: no top-k launched to device memory");
    }
    const uint32_t T = hist->block_tokens;
    const uint32_t L = hist->n_layers;
    int st = check_pool(ctx, pool, L, T, hist->n_embd_k, hist->n_embd_v, true);
    if (st != KVMEM_HIP_OK) {
        return st;
    }
    const uint64_t krow = kvmem_hip_row_size(pool->type_k, pool->n_embd_k);
    const uint64_t vrow = kvmem_hip_row_size(pool->type_v, pool->n_embd_v);
    const uint32_t cap = hist->capacity_blocks ? hist->capacity_blocks : hist->n_blocks;
    XfParams xp;
    st = resolve_xf(ctx, pool, hist->n_embd_k, hist->n_embd_v, true, xp);
    if (st != KVMEM_HIP_OK) {
        return st;
    }
    const uint32_t n_theta = xp.n_rot / 2;
    if ((pool->xf && pool->xf->pos0) || pool->n_slots > kPlanMaxSlots || max_sel == 0 || max_sel > kPlanMaxSel ||
        max_sel > pool->n_slots || n_res > pool->n_slots || T == 0 || T > 65535u || krow % 16 || vrow % 16 ||
        hist->n_embd_k % 32 || hist->n_embd_v % 32 || !aligned16(hist->k) || !aligned16(hist->v) ||
        cap < hist->n_blocks) {
        return fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "reselect_device: pool or history outside the device plan");
    }
    for (uint32_t r = 0; r < n_res; ++r) {
        if (res_slot[r] >= pool->n_slots || res_block[r] >= hist->n_blocks ||
            (r > 0 && (res_block[r] <= res_block[r - 1] || res_slot[r] <= res_slot[r - 1]))) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID, "reselect_device: resident blocks must ascend in id and slot");
        }
    }
    const uint32_t max_segs = max_sel;  // a move per segment at most
    const uint32_t max_saves = max_sel / kChainSeg + 1;
    const uint32_t ops_per = kPlanSaveOpsPer(L);
    auto up256 = [](size_t x) { return (x + 255) & ~size_t{255}; };
    const size_t off_stage = 256;
    const size_t theta_dst = 16 * size_t{L} + 16 * size_t{max_sel};  // in the stage table
    const size_t off_chain = up256(off_stage + theta_dst + 4 * size_t{n_theta});
    const size_t off_saves = up256(off_chain + 16 * size_t{L} + 4 * size_t{seg_record_words<uint16_t>()} * max_segs);
    const size_t plan_bytes = off_saves + sizeof(CopyOpDev) * size_t{ops_per} * max_saves;
    const uint64_t kspan = krow * T;
    const uint64_t vspan = vrow * T;
    const uint64_t per_move = (kspan + vspan) * L;
    (void) hipSetDevice(ctx->device);
    if (!ensure_dev(ctx, ctx->plan, plan_bytes, "reselect_device plan") ||
        !ensure_pin(ctx, ctx->plan_counts, sizeof(uint32_t) * kPlanCounts, "reselect_device counts",
                    hipHostMallocCoherent | hipHostMallocMapped) ||
        !ensure_dev(ctx, ctx->move_scratch, per_move * max_saves, "reselect_device scratch")) {
        return KVMEM_HIP_ERR_NOMEM;
    }
    void *counts_dev = nullptr;
    if (!hip_ok(ctx, hipHostGetDevicePointer(&counts_dev, ctx->plan_counts.ptr, 0), "reselect_device counts mapping")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    std::memset(ctx->plan_counts.ptr, 0, sizeof(uint32_t) * kPlanCounts);
    // the pool's layer pointers (K, then V), the resident table, then the
    // RoPE frequencies of a transformed pool
    const size_t theta_src = 16 * size_t{L} + 8 * size_t{n_res};
    std::vector<uint8_t> tab(theta_src + 4 * size_t{n_theta});
    std::memcpy(tab.data(), pool->k_layers, 8 * size_t{L});
    std::memcpy(tab.data() + 8 * size_t{L}, pool->v_layers, 8 * size_t{L});
    if (n_res) {
        std::memcpy(tab.data() + 16 * size_t{L}, res_block, 4 * size_t{n_res});
        std::memcpy(tab.data() + 16 * size_t{L} + 4 * size_t{n_res}, res_slot, 4 * size_t{n_res});
    }
    if (n_theta) {
        std::memcpy(tab.data() + theta_src, pool->xf->theta, 4 * size_t{n_theta});
    }
    LaunchTables lt;
    if (!stage_tables(ctx, tab.data(), tab.size(), lt, "reselect_device resident table")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    uint8_t *plan = static_cast<uint8_t *>(ctx->plan.ptr);
    uint8_t *scratch = static_cast<uint8_t *>(ctx->move_scratch.ptr);
    PlanParams pp{};
    pp.sel = static_cast<const uint32_t *>(ctx->topk_dev.ptr);
    pp.plan = plan;
    pp.counts_host = static_cast<uint32_t *>(counts_dev);
    pp.scratch = scratch;
    pp.tables = lt.dev;
    pp.kspan = kspan;
    pp.vspan = vspan;
    pp.entry_bytes = per_move;
    pp.off_stage = static_cast<uint32_t>(off_stage);
    pp.off_chain = static_cast<uint32_t>(off_chain);
    pp.off_saves = static_cast<uint32_t>(off_saves);
    pp.n_res = n_res;
    pp.n_slots = pool->n_slots;
    pp.n_blocks = hist->n_blocks;
    pp.T = T;
    pp.last_T = hist->last_block_tokens;
    pp.first_T = (hist->n_blocks == 1 && hist->last_block_tokens) ? hist->last_block_tokens : T;
    pp.n_theta = n_theta;
    pp.theta_src = static_cast<uint32_t>(theta_src);
    pp.theta_dst = static_cast<uint32_t>(theta_dst);
    pp.dirty = dirty;
    pp.L = L;
    pp.max_sel = max_sel;
    pp.max_saves = max_saves;
    ctx->plan_row_bytes = (krow + vrow) * L;
    ctx->plan_save_bytes = per_move;
    if (injected_fail(ctx, KVMEM_HIP_FAIL_LAUNCH, "reselect_device plan launch")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    {
        PerfScope planned(ctx, kPerfPlan);
        plan_kernel<<<1, kPlanThreads, 0, ctx->stream>>>(pp, lt.args);
        if (!hip_ok(ctx, hipGetLastError(), "reselect_device plan launch")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        planned.ok();
    }
    const uint32_t *counts = reinterpret_cast<const uint32_t *>(plan);
    // slot saves, then the chain walk
    PerfScope timed(ctx, kPerfLayout);
    if (!launch_dev_copies(ctx, reinterpret_cast<const CopyOpDev *>(plan + off_saves), counts + kPlanSaveOps,
                           ops_per * max_saves, "reselect_device saves")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    ChainParams cp{};
    cp.tables = plan + off_chain;
    cp.scratch = scratch;
    cp.dcount = counts + kPlanSegs;
    cp.kspan = kspan;
    cp.vspan = vspan;
    cp.entry_bytes = per_move;
    cp.krow16 = static_cast<uint32_t>(krow / 16);
    cp.vrow16 = static_cast<uint32_t>(vrow / 16);
    cp.L = L;
    cp.T = T;
    cp.vec_per_layer = T * (cp.krow16 + cp.vrow16);
    cp.max_segs = max_segs;
    const uint64_t nvec = static_cast<uint64_t>(L) * cp.vec_per_layer;
    if (nvec > 0x7fffffffu) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "reselect_device: slot too large");
    }
    if (injected_fail(ctx, KVMEM_HIP_FAIL_LAUNCH, "reselect_device chain launch")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    // up to kChainRows segments run side by side, one per grid row; more
    // take turns (a row's next segment waits for its stores)
    const dim3 cgrid(static_cast<uint32_t>((nvec + 255) / 256), std::min<uint32_t>(kChainRows, max_segs));
    move_chain_kernel<uint16_t><<<cgrid, 256, 0, ctx->stream>>>(cp, kNoArgTables);
    if (!hip_ok(ctx, hipGetLastError(), "reselect_device chain launch")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    timed.ok();
    ctx->plan_stage_off = off_stage;
    ctx->plan_theta_off = static_cast<uint32_t>(theta_dst);
    ctx->plan_max_sel = max_sel;
    return KVMEM_HIP_OK;
}

// The stage-in of the last device plan's n_staged blocks, launched by the
// host once it knows the count (the plan kernel wrote their items to the
// plan's stage table on the device): one workgroup per chunk, as the other
// stage-ins.
int kvmem_hip_reselect_device_stagein(kvmem_hip_ctx *ctx, const kvmem_hip_history *hist,
                                      const kvmem_hip_pool *pool, uint32_t n_staged) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (!hist || !hist->k || !hist->v || !pool || !pool->v_layers || (pool->xf && pool->xf->pos0) ||
        !ctx->plan.ptr || !ctx->plan_stage_off) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "reselect_device_stagein: no device plan");
    }
    if (n_staged > ctx->plan_max_sel || ctx->plan_max_sel > pool->n_slots) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "reselect_device_stagein: more blocks than the plan holds");
    }
    if (n_staged == 0) {
        return KVMEM_HIP_OK;
    }
    const uint32_t T = hist->block_tokens;
    const uint32_t L = hist->n_layers;
    const uint32_t cap = hist->capacity_blocks ? hist->capacity_blocks : hist->n_blocks;
    XfParams xp;
    const int xst = resolve_xf(ctx, pool, hist->n_embd_k, hist->n_embd_v, true, xp);
    if (xst != KVMEM_HIP_OK) {
        return xst;
    }
    JobTables jt;
    jt.tables.dev = static_cast<const uint8_t *>(ctx->plan.ptr) + ctx->plan_stage_off;
    jt.items_off = 16u * L;
    jt.theta_off = ctx->plan_theta_off;  // the plan kernel copied the RoPE frequencies there
    const uint64_t bk = static_cast<uint64_t>(T) * hist->n_embd_k * 2u;
    const uint64_t bv = static_cast<uint64_t>(T) * hist->n_embd_v * 2u;
    const BlockSource sk = make_block_source(pool->type_k, static_cast<const uint8_t *>(hist->k), bk, bk * cap, jt,
                                             L, T, hist->n_embd_k, 0, xp, true);
    const BlockSource sv = make_block_source(pool->type_v, static_cast<const uint8_t *>(hist->v), bv, bv * cap, jt,
                                             L, T, hist->n_embd_v, 0, xp, false);
    (void) hipSetDevice(ctx->device);
    PerfLaunchScope timed(ctx, kPerfSet);  // one launch: the events ride on it
    const int st = launch_block_job(ctx, pool->type_k, sk, pool->type_v, &sv, n_staged, xp, kNoArgTables);
    if (st == KVMEM_HIP_OK) {
        timed.ok();
    }
    return st;
}

// The last device plan's counts (kPlanCounts words: staged, moves,
// segments, saves, save copies, selected, error, moved rows), once the
// stream has drained; its moved and saved bytes join the copy counter.
int kvmem_hip_reselect_device_counts(kvmem_hip_ctx *ctx, uint32_t *out, uint32_t n) {
    if (!ctx || !out || !ctx->plan_counts.ptr) {
        return KVMEM_HIP_ERR_INVALID;
    }
    const uint32_t *c = static_cast<const uint32_t *>(ctx->plan_counts.ptr);
    for (uint32_t i = 0; i < n && i < kPlanCounts; ++i) {
        out[i] = __atomic_load_n(c + i, __ATOMIC_ACQUIRE);
    }
    // the saves' copy launch and the chain walk
    note_xfer(ctx, kXferD2D, static_cast<uint64_t>(c[kPlanSaves]) * ctx->plan_save_bytes, c[kPlanSaves] ? 1 : 0);
    note_xfer(ctx, kXferD2D, static_cast<uint64_t>(c[kPlanRows]) * ctx->plan_row_bytes, c[kPlanRows] ? 1 : 0);
    return KVMEM_HIP_OK;
}

}  // extern "C"

namespace kvmem_hip {

// Exhaustive device check of scale_div127 and scale_recip against the IEEE
// quotients: one thread per float bit pattern of the chunk.
__global__ __launch_bounds__(256) void check_scale_kernel(uint32_t base, uint32_t n, int which,
                                                          unsigned long long *bad) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) {
        return;
    }
    const float x = __uint_as_float(base + i);
    const float got = which == 0 ? scale_div127(x) : scale_recip(x);
    const float want = which == 0 ? x / 127.0f : 1.0f / x;
    if (__float_as_uint(got) != __float_as_uint(want)) {
        atomicAdd(bad, 1ull);
    }
}

}  // namespace kvmem_hip

extern "C" int kvmem_hip_check_scale_arith(kvmem_hip_ctx *ctx, uint64_t *div127_mismatches,
                                           uint64_t *recip_mismatches) {
    if (!ctx || !div127_mismatches || !recip_mismatches) {
        return KVMEM_HIP_ERR_INVALID;
    }
    (void) hipSetDevice(ctx->device);
    unsigned long long *bad = nullptr;
    if (!hip_ok(ctx, hipMalloc(&bad, 2 * sizeof(unsigned long long)), "check_scale_arith alloc")) {
        return KVMEM_HIP_ERR_NOMEM;
    }
    int rc = KVMEM_HIP_OK;
    if (!hip_ok(ctx, hipMemsetAsync(bad, 0, 2 * sizeof(unsigned long long), ctx->stream), "check_scale_arith")) {
        rc = KVMEM_HIP_ERR_RUNTIME;
    }
    // division: every non-negative finite float (zero and subnormals too);
    // reciprocal: normal floats of either sign with |x| <= 2^126
    const struct { uint32_t lo, hi; int which; } ranges[] = {
        {0x00000000u, 0x7f800000u, 0}, {0x00800000u, 0x7e800001u, 1}, {0x80800000u, 0xfe800001u, 1}};
    constexpr uint32_t kChunk = 1u << 26;
    for (const auto &r : ranges) {
        for (uint32_t b = r.lo; rc == KVMEM_HIP_OK && b < r.hi;) {
            const uint32_t n = (r.hi - b) < kChunk ? (r.hi - b) : kChunk;
            check_scale_kernel<<<(n + 255) / 256, 256, 0, ctx->stream>>>(b, n, r.which, bad + r.which);
            if (!hip_ok(ctx, hipGetLastError(), "check_scale_arith launch")) {
                rc = KVMEM_HIP_ERR_RUNTIME;
            }
            b += n;
        }
    }
    unsigned long long h[2] = {0, 0};
    if (rc == KVMEM_HIP_OK &&
        !hip_ok(ctx, hipMemcpyAsync(h, bad, sizeof(h), hipMemcpyDeviceToHost, ctx->stream), "check_scale_arith") ) {
        rc = KVMEM_HIP_ERR_RUNTIME;
    }
    if (rc == KVMEM_HIP_OK && !hip_ok(ctx, hipStreamSynchronize(ctx->stream), "check_scale_arith sync")) {
        rc = KVMEM_HIP_ERR_RUNTIME;
    }
    (void) hipFree(bad);
    *div127_mismatches = h[0];
    *recip_mismatches = h[1];
    return rc;
}
