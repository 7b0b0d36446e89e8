// GGUF weights on the GPU: ggml's Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q4_0, Q4_1, Q5_0, Q5_1 and Q8_0
// blocks decoded to fp32, Q4_K
// blocks rearranged into the ASDSL Q4_K variant that asdsl_gemv_q4km_q8 reads,
// and fp32 weights quantized to symmetric group-wise Q4 the way the
// reference requantizes GGUF projections (experiments/phi4_cpu_run.py:1437-1466:
// quantize_weights(bits=4, symmetric) from asdsl/quantization/core.py:358-420,
// bias = -7.5 * scale).
//
// The reference decodes K-quant blocks with the gguf package
// (asdsl/io/gguf_loader.py:150-181, gguf.quants.dequantize), which follows
// ggml's block layouts:
//   Q4_K, 144 bytes per 256 weights: fp16 d | fp16 dmin | 12 bytes holding
//     eight 6-bit scales and eight 6-bit mins | 128 bytes of nibbles.  Bytes
//     0-3 of the 12 hold scale j (low 6 bits) and bits 4-5 of scale j+4 (top
//     2 bits); bytes 4-7 the same for the mins; bytes 8-11 hold the low 4
//     bits of scale j+4 (low nibble) and of min j+4 (high nibble).  Nibble
//     byte 32c+l holds weight l of sub-block 2c (low nibble) and of
//     sub-block 2c+1 (high nibble).  w = (d*sc)*q - (dmin*m).
//   Q6_K, 210 bytes per 256 weights: 128 bytes of low nibbles, 64 bytes of
//     2-bit high parts, 16 int8 scales (one per 16 weights), fp16 d.  Each
//     half of 128 weights uses 64 low-nibble bytes, 32 high-part bytes and 8
//     scales: weight 32k+l (k = 0..3, l = 0..31) is the low (k < 2) or high
//     nibble of low byte l + 32(k&1), with bits 2k..2k+1 of high byte l on
//     top, minus 32, times (d * scale[l/16 + 2k]).
// Products and differences are formed one rounding at a time, in numpy's
// order, so the outputs are the gguf package's float32 values.
#include <hip/hip_fp16.h>

#include "abi_util.hpp"
#include "device_common.hpp"

namespace asdsl {
namespace {

constexpr int kGgufThreads = 256;
constexpr int kQ4kBytes = 144;
constexpr int kQ6kBytes = 210;
constexpr int kQ5kBytes = 176;
constexpr int kQ80Bytes = 34;
constexpr int kQ2kBytes = 84;
constexpr int kQ3kBytes = 110;

__device__ __forceinline__ float half_bits(uint32_t bits) {
    return __half2float(__ushort_as_half(static_cast<unsigned short>(bits & 0xFFFFu)));
}

// 6-bit scale and min of sub-block j of a ggml Q4_K block (s = its 12 bytes).
__device__ __forceinline__ void q4k_scale_min(const uint8_t (&s)[12], int j, int& sc, int& m) {
    if (j < 4) {
        sc = s[j] & 63;
        m = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

__device__ __forceinline__ void load_q4k_head(const uint8_t* blk, float& d, float& dmin, uint8_t (&s)[12]) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(blk);
    const uint32_t h = w[0];
    d = half_bits(h);
    dmin = half_bits(h >> 16);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const uint32_t v = w[1 + i];
#pragma unroll
        for (int b = 0; b < 4; ++b) s[4 * i + b] = static_cast<uint8_t>(v >> (8 * b));
    }
}

// ggml Q4_K -> fp32: 32 lanes per block, lane l writes weights 8l..8l+7
// (sub-block l/4, two float4 stores; consecutive lanes, consecutive bytes).
__global__ __launch_bounds__(kGgufThreads) void dequant_q4k_kernel(const uint8_t* __restrict__ blocks,
                                                                   float4* __restrict__ out, size_t n_blocks) {
    const size_t t = static_cast<size_t>(blockIdx.x) * kGgufThreads + threadIdx.x;
    const size_t b = t / 32;
    if (b >= n_blocks) return;
    const int l = static_cast<int>(t % 32);
    const uint8_t* blk = blocks + b * kQ4kBytes;
    float d, dmin;
    uint8_t s[12];
    load_q4k_head(blk, d, dmin, s);
    const int j = l / 4;
    int sc, m;
    q4k_scale_min(s, j, sc, m);
    const float d1 = __fmul_rn(d, static_cast<float>(sc));
    const float m1 = __fmul_rn(dmin, static_cast<float>(m));
    const uint2 raw = *reinterpret_cast<const uint2*>(blk + 16 + 32 * (j / 2) + 8 * (l % 4));
    const int shift = (j & 1) * 4;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t word = i < 4 ? raw.x : raw.y;
        const int q = (word >> (8 * (i % 4) + shift)) & 0x0F;
        v[i] = __fsub_rn(__fmul_rn(d1, static_cast<float>(q)), m1);
    }
    out[t * 2] = make_float4(v[0], v[1], v[2], v[3]);
    out[t * 2 + 1] = make_float4(v[4], v[5], v[6], v[7]);
}

// ggml Q6_K -> fp32: 32 lanes per block, lane l writes weights 8l..8l+7.
// Blocks are 210 bytes (2-byte aligned), read bytewise.
__global__ __launch_bounds__(kGgufThreads) void dequant_q6k_kernel(const uint8_t* __restrict__ blocks,
                                                                   float4* __restrict__ out, size_t n_blocks) {
    const size_t t = static_cast<size_t>(blockIdx.x) * kGgufThreads + threadIdx.x;
    const size_t b = t / 32;
    if (b >= n_blocks) return;
    const int l = static_cast<int>(t % 32);
    const uint8_t* blk = blocks + b * kQ6kBytes;
    const int h = l / 16;       // half of 128 weights
    const int e0 = 8 * (l % 16);  // first weight of the lane within the half
    const int k = e0 / 32;      // which of the four 32-weight quarters
    const int l0 = e0 % 32;
    const uint8_t* ql = blk + 64 * h + l0 + 32 * (k & 1);
    const uint8_t* qh = blk + 128 + 32 * h + l0;
    const int8_t scale = static_cast<int8_t>(blk[192 + 8 * h + l0 / 16 + 2 * k]);
    const float d = half_bits(static_cast<uint32_t>(blk[208]) | (static_cast<uint32_t>(blk[209]) << 8));
    const float ds = __fmul_rn(d, static_cast<float>(scale));
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int lo = k < 2 ? (ql[i] & 0x0F) : (ql[i] >> 4);
        const int hi = (qh[i] >> (2 * k)) & 3;
        v[i] = __fmul_rn(ds, static_cast<float>((lo | (hi << 4)) - 32));
    }
    out[t * 2] = make_float4(v[0], v[1], v[2], v[3]);
    out[t * 2 + 1] = make_float4(v[4], v[5], v[6], v[7]);
}

// ggml Q5_K -> fp32: 32 lanes per block, lane l writes weights 8l..8l+7 of
// sub-block j = l/4.  A block is 176 bytes (16-byte aligned blocks keep
// every field's offset a multiple of 4): fp16 d | fp16 dmin | the Q4_K
// 12-byte scale/min field | 32 bytes of high bits | 128 bytes of low
// nibbles.  Weight 32j + i (i < 32) takes the low (even j) or high (odd j)
// nibble of byte 48 + 32*(j/2) + i and bit j of byte 16 + i as its fifth
// bit: w = (d*sc)*q - (dmin*m), q in 0..31.
__global__ __launch_bounds__(kGgufThreads) void dequant_q5k_kernel(const uint8_t* __restrict__ blocks,
                                                                   float4* __restrict__ out, size_t n_blocks) {
    const size_t t = static_cast<size_t>(blockIdx.x) * kGgufThreads + threadIdx.x;
    const size_t b = t / 32;
    if (b >= n_blocks) return;
    const int l = static_cast<int>(t % 32);
    const uint8_t* blk = blocks + b * kQ5kBytes;
    float d, dmin;
    uint8_t s[12];
    load_q4k_head(blk, d, dmin, s);
    const int j = l / 4;
    int sc, m;
    q4k_scale_min(s, j, sc, m);
    const float d1 = __fmul_rn(d, static_cast<float>(sc));
    const float m1 = __fmul_rn(dmin, static_cast<float>(m));
    const int i0 = 8 * (l % 4);
    const uint2 lo = *reinterpret_cast<const uint2*>(blk + 48 + 32 * (j / 2) + i0);
    const uint2 hi = *reinterpret_cast<const uint2*>(blk + 16 + i0);
    const int shift = (j & 1) * 4;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t lw = i < 4 ? lo.x : lo.y;
        const uint32_t hw = i < 4 ? hi.x : hi.y;
        const int q = static_cast<int>(((lw >> (8 * (i % 4) + shift)) & 0x0Fu) |
                                       (((hw >> (8 * (i % 4) + j)) & 1u) << 4));
        v[i] = __fsub_rn(__fmul_rn(d1, static_cast<float>(q)), m1);
    }
    out[t * 2] = make_float4(v[0], v[1], v[2], v[3]);
    out[t * 2 + 1] = make_float4(v[4], v[5], v[6], v[7]);
}

// ggml Q8_0 -> fp32: 34 bytes per 32 weights, fp16 d then 32 int8 codes;
// w = code * d.  One thread per 8 weights, bytes read one at a time (the
// blocks are 2-byte aligned).
__global__ __launch_bounds__(kGgufThreads) void dequant_q8_0_kernel(const uint8_t* __restrict__ blocks,
                                                                    float4* __restrict__ out, size_t n_blocks) {
    const size_t t = static_cast<size_t>(blockIdx.x) * kGgufThreads + threadIdx.x;
    const size_t b = t / 4;
    if (b >= n_blocks) return;
    const uint8_t* blk = blocks + b * kQ80Bytes;
    const float d = half_bits(static_cast<uint32_t>(blk[0]) | (static_cast<uint32_t>(blk[1]) << 8));
    const uint8_t* q = blk + 2 + 8 * (t % 4);
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __fmul_rn(static_cast<float>(static_cast<int8_t>(q[i])), d);
    out[t * 2] = make_float4(v[0], v[1], v[2], v[3]);
    out[t * 2 + 1] = make_float4(v[4], v[5], v[6], v[7]);
}

// ggml's legacy 32-weight blocks -> fp32, one thread per 8 weights (bytes
// read one at a time: the blocks are 2-byte aligned).  Nibble byte j holds
// weight j (low nibble) and weight j + 16 (high nibble); the Q5 forms add a
// little-endian 32-bit word whose bit i is weight i's fifth bit.
//   Q4_0: fp16 d | 16 B nibbles, w = (q - 8) * d                        (18 B)
//   Q4_1: fp16 d | fp16 m | 16 B nibbles, w = d * q + m                 (20 B)
//   Q5_0: fp16 d | 4 B high bits | 16 B nibbles, w = (q - 16) * d       (22 B)
//   Q5_1: fp16 d | fp16 m | 4 B high bits | 16 B nibbles, w = d * q + m (24 B)
// The offset forms round the product and then the sum, as numpy does.
template <int BYTES>
__global__ __launch_bounds__(kGgufThreads) void dequant_legacy_kernel(const uint8_t* __restrict__ blocks,
                                                                      float4* __restrict__ out, size_t n_blocks) {
    constexpr bool kMin = BYTES == 20 || BYTES == 24;
    constexpr bool kHigh = BYTES == 22 || BYTES == 24;
    constexpr int kHighAt = kMin ? 4 : 2;
    constexpr int kCodesAt = kHighAt + (kHigh ? 4 : 0);
    const size_t t = static_cast<size_t>(blockIdx.x) * kGgufThreads + threadIdx.x;
    const size_t b = t / 4;
    if (b >= n_blocks) return;
    const int part = static_cast<int>(t % 4);  // weights 8 * part .. 8 * part + 7
    const uint8_t* blk = blocks + b * BYTES;
    auto rd16 = [&](int at) { return static_cast<uint32_t>(blk[at]) | (static_cast<uint32_t>(blk[at + 1]) << 8); };
    const float d = half_bits(rd16(0));
    const float m = kMin ? half_bits(rd16(2)) : 0.0f;
    const uint32_t qh = kHigh ? rd16(kHighAt) | (rd16(kHighAt + 2) << 16) : 0u;
    const uint8_t* qs = blk + kCodesAt + 8 * (part & 1);
    const int shift = (part >> 1) * 4;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int wi = 8 * part + i;
        const int q = static_cast<int>(((qs[i] >> shift) & 0x0Fu) | (((qh >> wi) & 1u) << 4));
        if constexpr (kMin) v[i] = __fadd_rn(__fmul_rn(d, static_cast<float>(q)), m);
        else v[i] = __fmul_rn(static_cast<float>(q - (kHigh ? 16 : 8)), d);
    }
    out[t * 2] = make_float4(v[0], v[1], v[2], v[3]);
    out[t * 2 + 1] = make_float4(v[4], v[5], v[6], v[7]);
}

// ggml Q2_K and Q3_K -> fp32: 32 lanes per block, lane l writes weights
// 8l..8l+7.  Both place weight 128n + 32j + 16h + i (i < 16) in bits
// 2j..2j+1 of code byte 32n + 16h + i under scale 8n + 2j + h, so a lane's
// eight weights share one scale and one shift.
//   Q2_K (84 B): 16 scale bytes | 64 code bytes | fp16 d | fp16 dmin; scale
//     byte s: w = (d * (s & 15)) * q - dmin * (s >> 4).
//   Q3_K (110 B): 32 high-mask bytes | 64 code bytes | 12 bytes of sixteen
//     6-bit scales | fp16 d; q -= 4 unless bit 4n + j of mask byte 16h + i
//     is set; scale k: low 4 bits from byte k (k < 8, low nibble) or k - 8
//     (high nibble), top 2 bits from bits 2(k/4).. of byte 8 + k % 4;
//     w = (d * (scale - 32)) * q.
template <bool Q3>
__global__ __launch_bounds__(kGgufThreads) void dequant_q23k_kernel(const uint8_t* __restrict__ blocks,
                                                                    float4* __restrict__ out, size_t n_blocks) {
    constexpr int kBytes = Q3 ? kQ3kBytes : kQ2kBytes;
    const size_t t = static_cast<size_t>(blockIdx.x) * kGgufThreads + threadIdx.x;
    const size_t b = t / 32;
    if (b >= n_blocks) return;
    const int l = static_cast<int>(t % 32);
    const int n = l / 16, j = (l % 16) / 4, h = (l % 4) / 2, i0 = 8 * (l % 2);
    const int k = 8 * n + 2 * j + h;  // scale index
    const uint8_t* blk = blocks + b * kBytes;
    auto rd16 = [&](int at) { return static_cast<uint32_t>(blk[at]) | (static_cast<uint32_t>(blk[at + 1]) << 8); };
    const uint8_t* qs = blk + (Q3 ? 32 : 16) + 32 * n + 16 * h + i0;
    float v[8];
    if constexpr (Q3) {
        const uint8_t* sc = blk + 96;
        const int lo = k < 8 ? (sc[k] & 15) : (sc[k - 8] >> 4);
        const int hi = (sc[8 + k % 4] >> (2 * (k / 4))) & 3;
        const float dl = __fmul_rn(half_bits(rd16(108)), static_cast<float>((lo | (hi << 4)) - 32));
        const uint8_t* hm = blk + 16 * h + i0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int q = ((qs[i] >> (2 * j)) & 3) - (((hm[i] >> (4 * n + j)) & 1) ? 0 : 4);
            v[i] = __fmul_rn(dl, static_cast<float>(q));
        }
    } else {
        const uint8_t s = blk[k];
        const float dl = __fmul_rn(half_bits(rd16(80)), static_cast<float>(s & 15));
        const float ml = __fmul_rn(half_bits(rd16(82)), static_cast<float>(s >> 4));
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = __fsub_rn(__fmul_rn(dl, static_cast<float>((qs[i] >> (2 * j)) & 3)), ml);
    }
    out[t * 2] = make_float4(v[0], v[1], v[2], v[3]);
    out[t * 2 + 1] = make_float4(v[4], v[5], v[6], v[7]);
}

// ggml Q4_K -> ASDSL Q4_K variant (asdsl/kernels/native/gemv_q4_avx2.cpp:78-120,
// 283-420: fp16 d | fp16 dmin | sixteen 6-bit entries LSB-first, scales then
// mins | sub-block j's 32 nibbles in bytes 16+16j.., low nibble first).
// Lossless: the same d, dmin, 6-bit scales, mins and 4-bit codes.  One
// thread per 16-byte piece of the output (9 a block: piece j < 8 is
// sub-block j's codes, piece 8 the head), so consecutive threads store
// consecutive bytes.
__global__ __launch_bounds__(kGgufThreads) void q4k_to_q4km_kernel(const uint8_t* __restrict__ src,
                                                                   uint8_t* __restrict__ dst, size_t n_blocks) {
    const size_t t = static_cast<size_t>(blockIdx.x) * kGgufThreads + threadIdx.x;
    const size_t b = t / 9;
    const int piece = static_cast<int>(t % 9);
    if (b >= n_blocks) return;
    const uint8_t* blk = src + b * kQ4kBytes;
    uint8_t* out = dst + b * kQ4kBytes;
    if (piece < 8) {
        const int j = piece;
        const uint4* chunk = reinterpret_cast<const uint4*>(blk + 16 + 32 * (j / 2));
        const uint4 a = chunk[0], c = chunk[1];
        const uint32_t in[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
        const int shift = (j & 1) * 4;
        uint32_t o[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < 16; ++i) {  // output byte i = codes 2i (low) and 2i+1 (high)
            const int k0 = 2 * i, k1 = 2 * i + 1;
            const uint32_t q0 = (in[k0 / 4] >> (8 * (k0 % 4) + shift)) & 0x0Fu;
            const uint32_t q1 = (in[k1 / 4] >> (8 * (k1 % 4) + shift)) & 0x0Fu;
            o[i / 4] |= (q0 | (q1 << 4)) << (8 * (i % 4));
        }
        *reinterpret_cast<uint4*>(out + 16 + 16 * j) = make_uint4(o[0], o[1], o[2], o[3]);
        return;
    }
    float d, dmin;
    uint8_t s[12];
    load_q4k_head(blk, d, dmin, s);
    uint32_t w[3] = {0u, 0u, 0u};
#pragma unroll
    for (int idx = 0; idx < 16; ++idx) {
        int sc, m;
        q4k_scale_min(s, idx % 8, sc, m);
        const uint32_t v = static_cast<uint32_t>(idx < 8 ? sc : m);
        const int bit = 6 * idx, word = bit / 32, off = bit % 32;
        w[word] |= v << off;
        if (off > 26) w[word + 1] |= v >> (32 - off);
    }
    *reinterpret_cast<uint4*>(out) = make_uint4(reinterpret_cast<const uint32_t*>(blk)[0], w[0], w[1], w[2]);
}

// fp32 -> symmetric Q4 (core.py:358-420 with symmetric=True, bits=4): per
// group of GS, scale = f16(max(amax, 1e-5) / 7.5), q = clip(rne(w /
// max(f32(scale), 1e-4) + 7.5), 0, 15), two codes a byte (low = even);
// scales out as f32(scale), biases as -7.5 * f32(scale).  GS/4 lanes per
// group, one float4 each.
template <int GS>
__global__ __launch_bounds__(kGgufThreads) void quantize_q4_sym_kernel(const float4* __restrict__ w,
                                                                       uint16_t* __restrict__ packed,
                                                                       float* __restrict__ scales,
                                                                       float* __restrict__ biases, size_t groups) {
    constexpr int kLanes = GS / 4;
    const size_t t = static_cast<size_t>(blockIdx.x) * kGgufThreads + threadIdx.x;
    const size_t g = t / kLanes;
    const bool live = g < groups;  // uniform over a group's lanes (kLanes divides the wave)
    const float4 v = live ? w[t] : make_float4(0.f, 0.f, 0.f, 0.f);
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
    for (int off = kLanes / 2; off > 0; off /= 2) amax = fmaxf(amax, __shfl_xor(amax, off));
    if (!live) return;
    const float scale = __fdiv_rn(fmaxf(amax, 1e-5f), 7.5f);
    const float sf = __half2float(__float2half_rn(scale));
    const float denom = fmaxf(sf, 1e-4f);
    auto code = [&](float x) {
        const float q = rintf(__fadd_rn(__fdiv_rn(x, denom), 7.5f));
        return static_cast<uint32_t>(fminf(fmaxf(q, 0.0f), 15.0f));
    };
    const uint32_t lo = code(v.x) | (code(v.y) << 4);
    const uint32_t hi = code(v.z) | (code(v.w) << 4);
    packed[t] = static_cast<uint16_t>(lo | (hi << 8));
    if (t % kLanes == 0) {
        scales[g] = sf;
        biases[g] = __fmul_rn(-7.5f, sf);
    }
}

unsigned grid_for(size_t threads) { return static_cast<unsigned>((threads + kGgufThreads - 1) / kGgufThreads); }

bool aligned(const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

asdsl_status check_k_blocks(const char* fn, int rows, int cols) {
    if (rows <= 0 || cols <= 0 || cols % 256 != 0) {
        set_error("%s: rows must be positive and cols a positive multiple of 256 (got %d x %d)", fn, rows, cols);
        return ASDSL_ERR_INVALID_ARGUMENT;
    }
    return ASDSL_OK;
}

}  // namespace
}  // namespace asdsl

using namespace asdsl;

extern "C" asdsl_status asdsl_dequant_gguf_q4k(const uint8_t* blocks, float* weights, int rows, int cols,
                                               asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(blocks && weights, "dequant_gguf_q4k: null pointer");
    const asdsl_status cs = check_k_blocks("dequant_gguf_q4k", rows, cols);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(aligned(blocks, 16) && aligned(weights, 16),
                    "dequant_gguf_q4k: blocks and weights must be 16-byte aligned");
    const size_t n = static_cast<size_t>(rows) * (cols / 256);
    return launch("dequant_q4k_kernel", dequant_q4k_kernel, dim3(grid_for(n * 32)), dim3(kGgufThreads), 0,
                  as_hip(stream), blocks, reinterpret_cast<float4*>(weights), n);
}

extern "C" asdsl_status asdsl_dequant_gguf_q6k(const uint8_t* blocks, float* weights, int rows, int cols,
                                               asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(blocks && weights, "dequant_gguf_q6k: null pointer");
    const asdsl_status cs = check_k_blocks("dequant_gguf_q6k", rows, cols);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(aligned(weights, 16), "dequant_gguf_q6k: weights must be 16-byte aligned");
    const size_t n = static_cast<size_t>(rows) * (cols / 256);
    return launch("dequant_q6k_kernel", dequant_q6k_kernel, dim3(grid_for(n * 32)), dim3(kGgufThreads), 0,
                  as_hip(stream), blocks, reinterpret_cast<float4*>(weights), n);
}

extern "C" asdsl_status asdsl_dequant_gguf_q5k(const uint8_t* blocks, float* weights, int rows, int cols,
                                               asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(blocks && weights, "dequant_gguf_q5k: null pointer");
    const asdsl_status cs = check_k_blocks("dequant_gguf_q5k", rows, cols);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(aligned(blocks, 16) && aligned(weights, 16),
                    "dequant_gguf_q5k: blocks and weights must be 16-byte aligned");
    const size_t n = static_cast<size_t>(rows) * (cols / 256);
    return launch("dequant_q5k_kernel", dequant_q5k_kernel, dim3(grid_for(n * 32)), dim3(kGgufThreads), 0,
                  as_hip(stream), blocks, reinterpret_cast<float4*>(weights), n);
}

extern "C" asdsl_status asdsl_dequant_gguf_q8_0(const uint8_t* blocks, float* weights, int rows, int cols,
                                                asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(blocks && weights, "dequant_gguf_q8_0: null pointer");
    if (rows <= 0 || cols <= 0 || cols % 32 != 0) {
        set_error("dequant_gguf_q8_0: rows must be positive and cols a positive multiple of 32 (got %d x %d)", rows,
                  cols);
        return ASDSL_ERR_INVALID_ARGUMENT;
    }
    ASDSL_CHECK_ARG(aligned(blocks, 2) && aligned(weights, 16),
                    "dequant_gguf_q8_0: blocks must be 2-byte and weights 16-byte aligned");
    const size_t n = static_cast<size_t>(rows) * (cols / 32);
    return launch("dequant_q8_0_kernel", dequant_q8_0_kernel, dim3(grid_for(n * 4)), dim3(kGgufThreads), 0,
                  as_hip(stream), blocks, reinterpret_cast<float4*>(weights), n);
}

namespace {

asdsl_status dequant_legacy(const char* fn, int bytes, const uint8_t* blocks, float* weights, int rows, int cols,
                            asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(blocks && weights, "%s: null pointer", fn);
    if (rows <= 0 || cols <= 0 || cols % 32 != 0) {
        set_error("%s: rows must be positive and cols a positive multiple of 32 (got %d x %d)", fn, rows, cols);
        return ASDSL_ERR_INVALID_ARGUMENT;
    }
    ASDSL_CHECK_ARG(aligned(blocks, 2) && aligned(weights, 16),
                    "%s: blocks must be 2-byte and weights 16-byte aligned", fn);
    const size_t n = static_cast<size_t>(rows) * (cols / 32);
    const dim3 grid(grid_for(n * 4)), block(kGgufThreads);
    hipStream_t s = as_hip(stream);
    float4* out = reinterpret_cast<float4*>(weights);
    switch (bytes) {
        case 18: return launch("dequant_legacy_kernel", dequant_legacy_kernel<18>, grid, block, 0, s, blocks, out, n);
        case 20: return launch("dequant_legacy_kernel", dequant_legacy_kernel<20>, grid, block, 0, s, blocks, out, n);
        case 22: return launch("dequant_legacy_kernel", dequant_legacy_kernel<22>, grid, block, 0, s, blocks, out, n);
        default: return launch("dequant_legacy_kernel", dequant_legacy_kernel<24>, grid, block, 0, s, blocks, out, n);
    }
}

asdsl_status dequant_q23k(const char* fn, bool q3, const uint8_t* blocks, float* weights, int rows, int cols,
                          asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(blocks && weights, "%s: null pointer", fn);
    const asdsl_status cs = check_k_blocks(fn, rows, cols);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(aligned(blocks, 2) && aligned(weights, 16),
                    "%s: blocks must be 2-byte and weights 16-byte aligned", fn);
    const size_t n = static_cast<size_t>(rows) * (cols / 256);
    const dim3 grid(grid_for(n * 32)), block(kGgufThreads);
    float4* out = reinterpret_cast<float4*>(weights);
    return q3 ? launch("dequant_q23k_kernel", dequant_q23k_kernel<true>, grid, block, 0, as_hip(stream), blocks, out,
                       n)
              : launch("dequant_q23k_kernel", dequant_q23k_kernel<false>, grid, block, 0, as_hip(stream), blocks,
                       out, n);
}

}  // namespace

extern "C" asdsl_status asdsl_dequant_gguf_q4_0(const uint8_t* blocks, float* weights, int rows, int cols,
                                                asdsl_stream_t stream) {
    return dequant_legacy("dequant_gguf_q4_0", 18, blocks, weights, rows, cols, stream);
}

extern "C" asdsl_status asdsl_dequant_gguf_q4_1(const uint8_t* blocks, float* weights, int rows, int cols,
                                                asdsl_stream_t stream) {
    return dequant_legacy("dequant_gguf_q4_1", 20, blocks, weights, rows, cols, stream);
}

extern "C" asdsl_status asdsl_dequant_gguf_q5_0(const uint8_t* blocks, float* weights, int rows, int cols,
                                                asdsl_stream_t stream) {
    return dequant_legacy("dequant_gguf_q5_0", 22, blocks, weights, rows, cols, stream);
}

extern "C" asdsl_status asdsl_dequant_gguf_q5_1(const uint8_t* blocks, float* weights, int rows, int cols,
                                                asdsl_stream_t stream) {
    return dequant_legacy("dequant_gguf_q5_1", 24, blocks, weights, rows, cols, stream);
}

extern "C" asdsl_status asdsl_dequant_gguf_q2k(const uint8_t* blocks, float* weights, int rows, int cols,
                                               asdsl_stream_t stream) {
    return dequant_q23k("dequant_gguf_q2k", false, blocks, weights, rows, cols, stream);
}

extern "C" asdsl_status asdsl_dequant_gguf_q3k(const uint8_t* blocks, float* weights, int rows, int cols,
                                               asdsl_stream_t stream) {
    return dequant_q23k("dequant_gguf_q3k", true, blocks, weights, rows, cols, stream);
}

extern "C" asdsl_status asdsl_repack_gguf_q4k_to_q4km(const uint8_t* gguf_blocks, uint8_t* q4km_blocks, int rows,
                                                      int cols, asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(gguf_blocks && q4km_blocks, "repack_gguf_q4k_to_q4km: null pointer");
    const asdsl_status cs = check_k_blocks("repack_gguf_q4k_to_q4km", rows, cols);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(aligned(gguf_blocks, 16) && aligned(q4km_blocks, 16),
                    "repack_gguf_q4k_to_q4km: both block arrays must be 16-byte aligned");
    const size_t n = static_cast<size_t>(rows) * (cols / 256);
    return launch("q4k_to_q4km_kernel", q4k_to_q4km_kernel, dim3(grid_for(n * 9)), dim3(kGgufThreads), 0,
                  as_hip(stream), gguf_blocks, q4km_blocks, n);
}

extern "C" asdsl_status asdsl_quantize_q4_symmetric(const float* weights, uint8_t* packed, float* scales,
                                                    float* biases, int rows, int cols, int group_size,
                                                    asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(weights && packed && scales && biases, "quantize_q4_symmetric: null pointer");
    ASDSL_CHECK_ARG(group_size == 32 || group_size == 64 || group_size == 128,
                    "quantize_q4_symmetric: group_size must be 32, 64 or 128");
    ASDSL_CHECK_ARG(rows > 0 && cols > 0 && cols % group_size == 0,
                    "quantize_q4_symmetric: rows must be positive and cols a positive multiple of group_size "
                    "(got %d x %d)", rows, cols);
    ASDSL_CHECK_ARG(aligned(weights, 16) && aligned(packed, 2) && aligned(scales, 4) && aligned(biases, 4),
                    "quantize_q4_symmetric: weights 16-byte, packed 2-byte, scales and biases 4-byte aligned");
    const size_t groups = static_cast<size_t>(rows) * (cols / group_size);
    const size_t threads = groups * (group_size / 4);
    const dim3 grid(grid_for(threads)), block(kGgufThreads);
    hipStream_t s = as_hip(stream);
    const float4* w = reinterpret_cast<const float4*>(weights);
    uint16_t* p = reinterpret_cast<uint16_t*>(packed);
    switch (group_size) {
        case 32: return launch("quantize_q4_sym_kernel", quantize_q4_sym_kernel<32>, grid, block, 0, s, w, p, scales,
                               biases, groups);
        case 64: return launch("quantize_q4_sym_kernel", quantize_q4_sym_kernel<64>, grid, block, 0, s, w, p, scales,
                               biases, groups);
        default: return launch("quantize_q4_sym_kernel", quantize_q4_sym_kernel<128>, grid, block, 0, s, w, p,
                               scales, biases, groups);
    }
}
