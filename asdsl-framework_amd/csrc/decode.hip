// One batch-1 decode step of a Phi-4-shaped model on the GPU: the glue around
// the preq2 GEMVs (embedding, RoPE + KV write + attention over an fp16 KV
// cache, greedy argmax) and the host driver that queues a whole token.
//
// Reference: UnifiedEngine::forward_token (asdsl/kernels/native/unified_engine.cpp:1339-1688)
//   with its helpers load_embed_row_f32 (181-197), rope_apply_inplace (768-801),
//   set_kv_cache (859-920), compute_attention_flash_q8 (922-1027),
//   argmax_f32_avx2 (207-233).  The cache is either the reference's form
//   (int8 codes with one fp32 scale per 64 dims; the current token's K/V are
//   quantized and dequantized before use, as the reference reads them back)
//   or fp16 rows (the current token's K/V rounded to fp16 before use).
//
// Per layer: qkv GEMV with residual add + RMSNorm in its prologue (layer 0:
// the embedding row itself), attention (RoPE, KV write, split partials),
// o_proj GEMV (below 512 positions it merges the partials in its prologue;
// beyond, a combine launch precedes it), gate_up GEMV with residual add +
// RMSNorm in its prologue and SwiGLU in its epilogue, down GEMV.  Five
// launches per layer below 512 positions, six beyond; then lm_head with the
// argmax and a one-thread finalize.  The token id and position live in
// device memory, so a captured graph of one step replays token after token
// with no host work.  The multi-token verify pass keeps a separate combine
// launch.
#include <hip/hip_fp16.h>

#include "abi_util.hpp"
#include "device_common.hpp"

namespace asdsl {
namespace {

constexpr int kHeadDim = 128;
constexpr int kSplit = 64;         // positions per attention workgroup
constexpr int kAttnThreads = 256;  // 4 waves x 4 positions per step
constexpr int kPartStride = kHeadDim + 2;  // m, l, acc[128]

__device__ __forceinline__ float h2f(uint16_t b) { return __half2float(__ushort_as_half(b)); }
__device__ __forceinline__ uint16_t f2h(float v) { return __half_as_ushort(__float2half_rn(v)); }

// One layer's KV cache as the attention kernels address it: rows of 128
// dims at [kv_head][position], either fp16 or int8 with one fp32 scale per
// 64 dims (scales [kv_head][position][2]; set_kv_cache,
// unified_engine.cpp:859-920).
struct KvCache {
    void* k;
    void* v;
    float* ks;  // int8 form only
    float* vs;
};

constexpr float kInv127 = 1.0f / 127.0f;

// Dims 8*dc .. 8*dc+7 of cache row `row` (kv_head * max_seq + position) in
// 16 bytes: fp16 as stored; int8 as the 8 codes, then the block's scale.
template <bool Q8>
__device__ __forceinline__ uint4 kv_load8(const void* base, const float* scales, size_t row, int dc) {
    if constexpr (Q8) {
        const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const int8_t*>(base) + row * kHeadDim + 8 * dc);
        return make_uint4(u.x, u.y, __float_as_uint(scales[row * 2 + (dc >> 3)]), 0u);
    } else {
        return *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + row * kHeadDim + 8 * dc);
    }
}

// kv_load8's 16 bytes as 8 floats: fp16 -> fp32, or float(code) * scale
// (compute_attention_flash_q8's dequantization, unified_engine.cpp:948-951).
template <bool Q8>
__device__ __forceinline__ void kv_unpack8(const uint4& raw, float (&r)[8]) {
    if constexpr (Q8) {
        const float sc = __uint_as_float(raw.z);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            r[e] = static_cast<float>(static_cast<int8_t>(raw.x >> (8 * e))) * sc;
            r[4 + e] = static_cast<float>(static_cast<int8_t>(raw.y >> (8 * e))) * sc;
        }
    } else {
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            r[2 * e] = h2f(static_cast<uint16_t>(w[e] & 0xFFFFu));
            r[2 * e + 1] = h2f(static_cast<uint16_t>(w[e] >> 16));
        }
    }
}

// set_kv_cache's rule on one 64-dim block held one value per lane of a wave:
// scale = amax * (1/127) if amax > 1e-12, else 1e-12; returns the code
// round-half-even(x * (1 / scale)) clamped to [-127, 127].
__device__ __forceinline__ int kv_q8_code(float x, float& scale) {
    float a = fabsf(x);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, kWave));
    scale = a > 1e-12f ? a * kInv127 : 1e-12f;
    const float inv = 1.0f / scale;
    const float q = __builtin_rintf(x * inv);
    return static_cast<int>(fminf(fmaxf(q, -127.0f), 127.0f));
}

// h[0:hidden] = embed[token] (fp16 -> fp32); also clears the argmax slot for
// this step's lm_head.  A token outside [0, vocab) reads row 0 (the host
// validates tokens; the device-side loop only produces argmax rows).
__global__ __launch_bounds__(256) void embed_kernel(const uint16_t* __restrict__ embed, const int* __restrict__ token,
                                                    float* __restrict__ h, int hidden, int vocab,
                                                    unsigned long long* __restrict__ amax) {
    const int t0 = *token;
    const int t = t0 >= 0 && t0 < vocab ? t0 : 0;
    const uint16_t* row = embed + static_cast<size_t>(t) * hidden;
    for (int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x); i < hidden;
         i += static_cast<int>(gridDim.x * blockDim.x))
        h[i] = h2f(row[i]);
    if (blockIdx.x == 0 && threadIdx.x == 0 && amax) *amax = 0ull;
}

ASDSL_TIMELINE_BUFFER

// Next token = the argmax row; position + 1.
__global__ void finalize_kernel(const unsigned long long* __restrict__ amax, int* __restrict__ token,
                                int* __restrict__ pos) {
    if (threadIdx.x == 0) {
        *token = static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(*amax));
        *pos += 1;
    }
}

// The end of a split's attention in a workgroup of NT threads: every lane
// holds its own running (m, l, acc) over the positions it scanned; the 16
// lanes of one position slot of one wave (a group) share m and l, and each
// holds acc for its 8 dims.  The NG = NT/16 groups merge in LDS in fixed
// order, with no cross-lane reduction: M = max_k m_k, e_k = exp(m_k - M) (0
// for a group that saw no position), acc = sum_k e_k acc_k, l = sum_k e_k l_k;
// writes (M, l, acc[128]) of head hh at part + hh * head_stride.  (Folding the
// slots of a wave first with swizzles and permutes measured ~40 % of the
// kernel: 5.4 against 2.0 us for its loads alone at ctx 128.)
template <int G, int NT>
__device__ __forceinline__ void merge_position_groups(const float (&m)[G], const float (&l)[G],
                                                      const float (&acc)[G][8], float (*gml)[G][2],
                                                      float (*gacc)[G][kHeadDim], float (*ge)[NT / 16],
                                                      float* __restrict__ part, size_t head_stride) {
#pragma clang fp contract(off)
    constexpr int NG = NT / 16;
    const int tid = static_cast<int>(threadIdx.x);
    const int k = tid >> 4;  // group: wave * 4 + position slot
    const int dc = tid & 15;
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
        float4* dst = reinterpret_cast<float4*>(&gacc[k][hh][8 * dc]);
        dst[0] = make_float4(acc[hh][0], acc[hh][1], acc[hh][2], acc[hh][3]);
        dst[1] = make_float4(acc[hh][4], acc[hh][5], acc[hh][6], acc[hh][7]);
    }
    if (dc == 0) {
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
            gml[k][hh][0] = m[hh];
            gml[k][hh][1] = l[hh];
        }
    }
    __syncthreads();
    if (tid < G * NG) {  // e_k of every (head, group)
        const int hh = tid / NG;
        const int kk = tid % NG;
        float M = gml[0][hh][0];
#pragma unroll
        for (int j = 1; j < NG; ++j) M = fmaxf(M, gml[j][hh][0]);
        const float mk = gml[kk][hh][0];
        ge[hh][kk] = mk == -INFINITY ? 0.0f : expf(mk - M);
    }
    __syncthreads();
    for (int e = tid; e < G * kHeadDim; e += NT) {
        const int hh = e / kHeadDim;
        const int d = e % kHeadDim;
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < NG; ++j) sum = fmaf(ge[hh][j], gacc[j][hh][d], sum);
        part[hh * head_stride + 2 + d] = sum;
    }
    if (tid < G) {
        float M = gml[0][tid][0];
#pragma unroll
        for (int j = 1; j < NG; ++j) M = fmaxf(M, gml[j][tid][0]);
        float L = 0.0f;
#pragma unroll
        for (int j = 0; j < NG; ++j) L = fmaf(ge[tid][j], gml[j][tid][1], L);
        float* pp = part + tid * head_stride;
        pp[0] = M;
        pp[1] = L;
    }
}

// Scores, split-local softmax and P.V of one split for the G query heads of a
// KV head, then the merge of the four waves: lane (wave, pg, dc) holds the
// K/V rows of positions p0 + 4*wave + pg + 16*it in kraw/vraw (dims
// 8*dc..+8) and its query chunks in qr; positions >= p1 are masked.  With
// NEW, position `pos` takes its K/V rows from kv_new (LDS) instead.  Writes
// (m, l, acc[128]) of head hh at part + hh * head_stride.
template <int G, bool NEW, bool Q8>
__device__ __forceinline__ void attn_split_core(const uint4 (&kraw)[kSplit / 16], const uint4 (&vraw)[kSplit / 16],
                                                const float (&qr)[G][8], int p0, int p1, int pos,
                                                const float (*kv_new)[kHeadDim], float (*gml)[G][2],
                                                float (*gacc)[G][kHeadDim], float (*ge)[kAttnThreads / 16],
                                                float* __restrict__ part, size_t head_stride) {
    // no implicit fused multiply-adds: the folded form's kernel computes the
    // same scores and weights and must round them alike
#pragma clang fp contract(off)
    constexpr int kIt = kSplit / 16;
    const int tid = static_cast<int>(threadIdx.x);
    const float inv_sqrt_d = 1.0f / sqrtf(static_cast<float>(kHeadDim));
    const int lane = tid & (kWave - 1);
    const int wave = tid >> 6;
    const int pg = lane >> 4;
    const int dc = lane & 15;
    auto row_of = [&](const uint4& raw, int which, int p, float (&r)[8]) {
        if (NEW && p == pos) {
#pragma unroll
            for (int e = 0; e < 8; ++e) r[e] = kv_new[which][8 * dc + e];
        } else {
            kv_unpack8<Q8>(raw, r);
        }
    };

    // scores of this lane's positions (the 16 lanes of a position all hold
    // it after the DPP sum); positions past the split are -inf
    float sr[kIt][G];
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
        const int p = p0 + wave * 4 + pg + 16 * it;
        float k8[8];
        row_of(kraw[it], 0, p, k8);
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) d = fmaf(qr[hh][e], k8[e], d);
            d += dpp<kDppQuadXor1>(d);  // sum over the 16 lanes of the position
            d += dpp<kDppQuadXor2>(d);
            d += dpp<kDppRowRor4>(d);
            d += dpp<kDppRowRor8>(d);
            sr[it][hh] = p < p1 ? d * inv_sqrt_d : -INFINITY;
        }
    }
    // this lane's max and exp-sum per head over its iterations; a lane with
    // no position keeps m = -inf and l = 0
    float m[G], l[G];
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
        float v = sr[0][hh];
#pragma unroll
        for (int it = 1; it < kIt; ++it) v = fmaxf(v, sr[it][hh]);
        m[hh] = v;  // this lane's positions (the 16 lanes of its slot agree)
    }
    float acc[G][8];
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
        l[hh] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[hh][e] = 0.0f;
    }
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
        const int p = p0 + wave * 4 + pg + 16 * it;
        float v8[8];
        row_of(vraw[it], 1, p, v8);
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
            const float w = p < p1 ? expf(sr[it][hh] - m[hh]) : 0.0f;
            l[hh] += w;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[hh][e] = fmaf(w, v8[e], acc[hh][e]);
        }
    }
    merge_position_groups<G, kAttnThreads>(m, l, acc, gml, gacc, ge, part, head_stride);
}

// int8 cache: the new position's rotated key and value (kv_new, fp32)
// become their codes.  Each of the four waves takes one 64-dim block (waves
// 0-1: the key's blocks, 2-3: the value's), leaves the dequantized values in
// kv_new (what a later step reads back) and, when `store`, writes the codes
// and the scale to cache row `row`.
// (called by the first four waves of a workgroup)
__device__ __forceinline__ void kv_quantize_new(float (*kv_new)[kHeadDim], const KvCache& kv, size_t row,
                                                bool store) {
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = tid >> 6;
    const int which = wave >> 1;
    const int d = (wave & 1) * kWave + (tid & (kWave - 1));
    float scale;
    const int q = kv_q8_code(kv_new[which][d], scale);
    kv_new[which][d] = static_cast<float>(q) * scale;
    if (store) {
        static_cast<int8_t*>(which ? kv.v : kv.k)[row * kHeadDim + d] = static_cast<int8_t>(q);
        if ((tid & (kWave - 1)) == 0) (which ? kv.vs : kv.ks)[row * 2 + (wave & 1)] = scale;
    }
}

// out[h][d] = sum_s e_s acc_s[d] / sum_s e_s l_s, e_s = exp(m_s - max m).
// Up to kCombineGroups groups of 128 threads each fold a contiguous run of
// splits (chunks of kChunk loads issued together, a running (max, sum,
// output) rescaled between chunks); with more than one group the runs are
// merged in LDS in split order.  One group when the splits fit one chunk.
// blockIdx.y = column c of a multi-token pass (position *pos_ptr + c; its
// partials and output follow column c - 1's); the decode step runs one column.
constexpr int kCombineGroups = 8;
constexpr int kCombineThreads = kCombineGroups * kHeadDim;
constexpr int kCombineChunk = 16;  // splits whose loads a group issues together

// Threads of a combine launch whose positions have at most max_ns splits:
// one group of 128 per kCombineChunk splits, so that no wave of the
// workgroup idles (the kernel's grouping, and with it its fp32 order,
// depends on the position's split count alone).
inline int combine_threads(int max_ns) {
    const int groups = (max_ns + kCombineChunk - 1) / kCombineChunk;
    return kHeadDim * (groups < 1 ? 1 : groups > kCombineGroups ? kCombineGroups : groups);
}

// IMG_GS (32 or 128): the head's 128 outputs of column c are also quantized
// into the o_proj batched GEMV's int8 image (image_store8, 16 chunks per
// head), and columns c >= ncols (the grid covers kImageCols columns) write
// that image's zero columns.
template <int IMG_GS>
__global__ __launch_bounds__(kCombineThreads) void attn_combine_kernel(const float* __restrict__ part,
                                                                      const int* __restrict__ pos_ptr,
                                                                      float* __restrict__ out, int nsplit,
                                                                      int max_seq, int pos_limit, int fold, int ncols,
                                                                      int form_tile, int form_splits,
                                                                      uint2* __restrict__ img,
                                                                      float2* __restrict__ fac,
                                                                      float* __restrict__ us) {
    constexpr int kChunk = kCombineChunk;
    constexpr int kHeadChunks = kHeadDim / 8;
    __shared__ float gml[kCombineGroups][2];
    __shared__ float go[kCombineGroups][kHeadDim];
    __shared__ float res_s[IMG_GS != 0 ? kHeadDim : 1];
    const int col = static_cast<int>(blockIdx.y);
    const int h = static_cast<int>(blockIdx.x);
    const int tid = static_cast<int>(threadIdx.x);
    const int d = tid % kHeadDim;
    const int g = tid / kHeadDim;
    // the first kHeadChunks lanes quantize the head's outputs (8 each)
    auto image_chunk = [&](const float (&v)[8]) {
        if constexpr (IMG_GS != 0) image_store8<IMG_GS>(v, h * kHeadChunks + tid, col, true, img, fac, us);
    };
    const float zeros[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (IMG_GS != 0 && col >= ncols) {
        if (tid < kHeadChunks) image_chunk(zeros);
        return;
    }
    const int pos = *pos_ptr + col;
    part += static_cast<size_t>(col) * gridDim.x * nsplit * kPartStride;
    out += static_cast<size_t>(col) * gridDim.x * kHeadDim;
    if (pos < 0 || pos >= max_seq || pos >= pos_limit) {  // no partials were written (see attn_decode_kernel)
        if (g == 0) out[static_cast<size_t>(h) * kHeadDim + d] = 0.0f;
        if (IMG_GS != 0 && tid < kHeadChunks) image_chunk(zeros);
        return;
    }
    // splits: form_splits > 0, the decode step's attention (pos / form_tile + 1
    // tiles in at most form_splits splits); otherwise one per kSplit positions
    const int nt = pos / (form_splits > 0 ? form_tile : kSplit) + 1;
    const int tps = form_splits > 0 ? (nt + form_splits - 1) / form_splits : 1;
    const int ns = (nt + tps - 1) / tps;
    if (ns <= fold) return;  // the consuming GEMV's prologue merges these splits itself
    const int tl_slot = col == 0 ? 6 : -1;
    ASDSL_TIMELINE_STAMP(tl_slot, h, 0);
    // groups with splits (the launch gives every one of them its 128 threads:
    // combine_threads of the most splits its positions can have)
    const int ng = min(kCombineGroups, (ns + kChunk - 1) / kChunk);
    const int per = (ns + ng - 1) / ng;
    const int s_begin = min(ns, g * per);
    const int s_end = min(ns, s_begin + per);
    const float* ph = part + static_cast<size_t>(h) * nsplit * kPartStride;
    float M = -INFINITY, L = 0.0f, o = 0.0f;
    for (int s0 = s_begin; s0 < s_end; s0 += kChunk) {  // uniform per group
        float mv[kChunk], lv[kChunk], av[kChunk];
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            const bool live = s0 + j < s_end;
            const float* pp = ph + static_cast<size_t>(live ? s0 + j : 0) * kPartStride;
            mv[j] = live ? pp[0] : -INFINITY;
            lv[j] = live ? pp[1] : 0.0f;
            av[j] = live ? pp[2 + d] : 0.0f;
        }
        float cm = M;
#pragma unroll
        for (int j = 0; j < kChunk; ++j) cm = fmaxf(cm, mv[j]);
        const float r = M == -INFINITY ? 0.0f : expf(M - cm);
        L *= r;
        o *= r;
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            if (s0 + j < s_end) {
                const float e = expf(mv[j] - cm);
                L = fmaf(e, lv[j], L);
                o = fmaf(e, av[j], o);
            }
        }
        M = cm;
    }
    ASDSL_TIMELINE_STAMP(tl_slot, h, 3);
    float res = 0.0f;  // group 0: the output of dimension d
    if (ng == 1) {     // uniform: group 0 holds every split
        res = o * (1.0f / L);
    } else {
        go[g][d] = o;
        if (d == 0) {
            gml[g][0] = M;
            gml[g][1] = L;
        }
        __syncthreads();
        if (g == 0) {
            float Mx = gml[0][0];
            for (int q = 1; q < ng; ++q) Mx = fmaxf(Mx, gml[q][0]);
            float sum = 0.0f, Ls = 0.0f;
            for (int q = 0; q < ng; ++q) {
                const float mq = gml[q][0];
                const float e = mq == -INFINITY ? 0.0f : expf(mq - Mx);
                sum = fmaf(e, go[q][d], sum);
                Ls = fmaf(e, gml[q][1], Ls);
            }
            res = sum * (1.0f / Ls);
        }
    }
    if (g == 0) out[static_cast<size_t>(h) * kHeadDim + d] = res;
    if constexpr (IMG_GS != 0) {
        if (g == 0) res_s[d] = res;
        __syncthreads();
        if (tid < kHeadChunks) {
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = res_s[8 * tid + e];
            image_chunk(v);
        }
    }
    ASDSL_TIMELINE_STAMP(tl_slot, h, 4);
}

// ------------------------------------------------------------ decode attention
// The decode step's attention.  Workgroup (s, kvh) of WAVES waves covers
// split s of the KV head's positions: tps consecutive tiles of tile = 4 *
// WAVES * KIT positions (a wave takes 4 positions per step, KIT steps a
// tile), at most max_splits splits, the next tile's K/V rows requested
// before the current tile is used and a running (max, sum, P.V) per lane;
// the lanes merge in LDS and the partial (m, l, acc) of each query head is
// stored.  Three forms, all with tiles of 64:
//   short (positions below 512; 4 waves, at most 8 splits of one tile): the
//     o_proj GEMV's prologue merges the splits (no combine launch);
//   long (up to 2048; 4 waves, at most 32 splits of one tile) and deep
//     (beyond; 8 waves, at most 32 splits of ceil(tiles / 32) tiles): the
//     combine kernel merges them.
// Against 64-position splits over the whole cache with a combine (the
// verify pass's form), these measured 1040 against 1081 us per 32-layer
// step at ctx 1024 and 1194 against 1218 at 4096 (fp16; int8 1039 against
// 1073 and 1203 against 1195): the launch covers only the splits its
// position range uses, and the combine folds at most 32 partials.  Capping
// at 8, 16, 48, 64 or 80 splits measured slower, as did 8 waves with tiles
// of 128 or 16 waves with tiles of 256.  A position outside the cache gives
// zero output.
constexpr int kMaxSplits = 32;  // partial rows reserved per query head
constexpr int kShortLimit = 512;
struct FoldForm {
    int waves, tile, max_splits;
};
constexpr FoldForm kShortForm{4, 64, 8};
constexpr FoldForm kLongForm{4, 64, kMaxSplits};
// Beyond 2048 positions a split holds several tiles: 8 waves per tile of 64
// (two steps each) shorten each wave's dependent chain and measured 1194
// against 1216 us per 32-layer step at ctx 4096 (int8 1203 against 1209 with
// 4 waves); with one tile per split (up to 2048) they measured slower (1048
// against 1043 at 1024), and 16 waves slower still.
constexpr FoldForm kDeepForm{8, 64, kMaxSplits};
constexpr int kDeepFrom = 2048;
static_assert(kShortForm.max_splits <= 8, "o_proj's prologue folds at most 8 splits");
static_assert(kShortForm.waves == kLongForm.waves && kShortForm.tile == kLongForm.tile &&
                  kDeepForm.tile == kLongForm.tile, "one tile size for the forms and the combine");

__host__ __device__ inline int attn_fold_tps(int pos, int tile, int max_splits) {
    const int nt = pos / tile + 1;
    return (nt + max_splits - 1) / max_splits;
}

__host__ __device__ inline int attn_fold_splits(int pos, int tile, int max_splits) {
    const int nt = pos / tile + 1;
    const int tps = (nt + max_splits - 1) / max_splits;
    return (nt + tps - 1) / tps;
}

// Positions below pos_limit take the short form when pos_limit <= 512.
bool attn_fold(int pos_limit) { return pos_limit <= kShortLimit; }

// Most splits any position below pos_limit uses (the launch's grid.x).
int attn_max_splits(int pos_limit, const FoldForm& f) {
    int best = 1;
    for (int nt = 1; (nt - 1) * f.tile < pos_limit; ++nt) {
        const int tps = (nt + f.max_splits - 1) / f.max_splits;
        best = max(best, (nt + tps - 1) / tps);
        if (best == f.max_splits) break;
    }
    return best;
}

template <int G, bool Q8, int WAVES, int KIT>
__global__ __launch_bounds__(WAVES * kWave) void attn_decode_kernel(
    const float* __restrict__ qkv, KvCache kv,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin, const int* __restrict__ pos_ptr,
    float* __restrict__ part, float* __restrict__ att, int n_heads, int n_kv, int max_seq, int rot_half,
    int max_splits, int pos_limit, uint32_t* __restrict__ flags) {
    constexpr int kThreads = WAVES * kWave;
    constexpr int kStep = 4 * WAVES;   // positions per step of all waves
    constexpr int kIt = KIT;           // steps per tile
    constexpr int kTile = kStep * kIt; // positions per tile
    __shared__ float q_s[G][kHeadDim];
    __shared__ float kv_new[2][kHeadDim];
    __shared__ float gml[kThreads / 16][G][2];
    __shared__ __align__(16) float gacc[kThreads / 16][G][kHeadDim];
    __shared__ float ge[G][kThreads / 16];
    const int s = static_cast<int>(blockIdx.x);
    const int kvh = static_cast<int>(blockIdx.y);
    const int tid = static_cast<int>(threadIdx.x);
    const int tl_wg = static_cast<int>(blockIdx.y * gridDim.x + blockIdx.x);
    ASDSL_TIMELINE_STAMP(4, tl_wg, 0);
    const int pos = *pos_ptr;
    // Outside the cache, or at or past the range the launch was shaped for
    // (its grid would not cover the position's splits): zero output, nothing
    // written to the cache, and the reason raised in *flags for the host.
    if (pos < 0 || pos >= max_seq || pos >= pos_limit) {
        if (s == 0)
            for (int e = tid; e < G * kHeadDim; e += kThreads) att[static_cast<size_t>(kvh * G) * kHeadDim + e] = 0.0f;
        if (flags && s == 0 && kvh == 0 && tid == 0)
            *flags |= pos < 0 || pos >= max_seq ? ASDSL_DECODE_FLAG_POS_RANGE : ASDSL_DECODE_FLAG_POS_LIMIT;
        return;
    }
    const int tps = attn_fold_tps(pos, kTile, max_splits);
    const int ns = attn_fold_splits(pos, kTile, max_splits);
    if (s >= ns) return;
    const int p0 = s * tps * kTile;
    const int p1 = min(p0 + tps * kTile, pos + 1);
    const int lane = tid & (kWave - 1);
    const int wave = tid >> 6;
    const int pg = lane >> 4;   // position within the wave's four
    const int dc = lane & 15;   // 8-dim chunk
    const size_t row0 = static_cast<size_t>(kvh) * max_seq;  // cache row of position 0

    // RoPE inputs of the G query heads and the new key (small, first), then
    // the first tile's K/V rows: loads complete in issue order.
    const float* cp = rope_cos + static_cast<size_t>(pos) * rot_half;
    const float* sp = rope_sin + static_cast<size_t>(pos) * rot_half;
    constexpr int kRope = ((G + 1) * kHeadDim + kThreads - 1) / kThreads;
    float rx[kRope][4];
#pragma unroll
    for (int r = 0; r < kRope; ++r) {
        const int e = tid + r * kThreads;
        const int hh = e / kHeadDim;
        const int d = e % kHeadDim;
        if (hh <= G) {
            const float* src = hh < G ? qkv + static_cast<size_t>(kvh * G + hh) * kHeadDim
                                      : qkv + static_cast<size_t>(n_heads + kvh) * kHeadDim;
            if (d < 2 * rot_half) {
                const int i = d < rot_half ? d : d - rot_half;
                rx[r][0] = src[i];
                rx[r][1] = src[i + rot_half];
                rx[r][2] = cp[i];
                rx[r][3] = sp[i];
            } else {
                rx[r][0] = src[d];
            }
        }
    }
    const float* vsrc = qkv + static_cast<size_t>(n_heads + n_kv + kvh) * kHeadDim;
    const float vnew = tid < kHeadDim ? vsrc[tid] : 0.0f;

    // Unconditional loads (positions past the split read the split's first
    // row; the row at `pos` is taken from LDS): no branch around a load, so
    // the rows stay in registers with every load in flight.
    auto load_tile = [&](int t0, uint4 (&kraw)[kIt], uint4 (&vraw)[kIt]) {
#pragma unroll
        for (int it = 0; it < kIt; ++it) {
            const int p = t0 + wave * 4 + pg + kStep * it;
            const size_t row = row0 + (p < p1 ? p : p0);
            kraw[it] = kv_load8<Q8>(kv.k, kv.ks, row, dc);
            vraw[it] = kv_load8<Q8>(kv.v, kv.vs, row, dc);
        }
    };
    uint4 ka[kIt], va[kIt], kb[kIt], vb[kIt];
    load_tile(p0, ka, va);

#pragma unroll
    for (int r = 0; r < kRope; ++r) {
        const int e = tid + r * kThreads;
        const int hh = e / kHeadDim;
        const int d = e % kHeadDim;
        if (hh <= G) {
            float val;
            if (d < 2 * rot_half) {
                const float xf = rx[r][0], xs = rx[r][1], c = rx[r][2], sn = rx[r][3];
                val = d < rot_half ? fmaf(xf, c, -(xs * sn)) : fmaf(xf, sn, xs * c);
            } else {
                val = rx[r][0];
            }
            if (hh < G) q_s[hh][d] = val;
            else kv_new[0][d] = Q8 ? val : h2f(f2h(val));
        }
    }
    if (tid < kHeadDim) kv_new[1][tid] = Q8 ? vnew : h2f(f2h(vnew));
    ASDSL_TIMELINE_STAMP(4, tl_wg, 1);
    __syncthreads();
    if constexpr (Q8) {
        if (wave < 4) kv_quantize_new(kv_new, kv, row0 + pos, pos >= p0 && pos < p1);
        __syncthreads();
    } else if (pos >= p0 && pos < p1 && tid < kHeadDim) {
        static_cast<uint16_t*>(kv.k)[(row0 + pos) * kHeadDim + tid] = f2h(kv_new[0][tid]);
        static_cast<uint16_t*>(kv.v)[(row0 + pos) * kHeadDim + tid] = f2h(kv_new[1][tid]);
    }
    float qr[G][8];
#pragma unroll
    for (int hh = 0; hh < G; ++hh)
#pragma unroll
        for (int e = 0; e < 8; ++e) qr[hh][e] = q_s[hh][8 * dc + e];

    // running state of this lane over its positions: max, exp-sum and P.V
    // (its 8 dims; the 16 lanes of its position slot share max and sum)
    const float inv_sqrt_d = 1.0f / sqrtf(static_cast<float>(kHeadDim));
    float m[G], l[G], acc[G][8];
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
        m[hh] = -INFINITY;
        l[hh] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[hh][e] = 0.0f;
    }
    auto row_of = [&](const uint4& raw, int which, int p, float (&r)[8]) {
        if (p == pos) {
#pragma unroll
            for (int e = 0; e < 8; ++e) r[e] = kv_new[which][8 * dc + e];
        } else {
            kv_unpack8<Q8>(raw, r);
        }
    };
    auto process_tile = [&](int t0, const uint4 (&kraw)[kIt], const uint4 (&vraw)[kIt]) {
#pragma clang fp contract(off)  // rounds as attn_split_core does
        float sr[kIt][G];
#pragma unroll
        for (int it = 0; it < kIt; ++it) {
            const int p = t0 + wave * 4 + pg + kStep * it;
            float k8[8];
            row_of(kraw[it], 0, p, k8);
#pragma unroll
            for (int hh = 0; hh < G; ++hh) {
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) d = fmaf(qr[hh][e], k8[e], d);
                d += dpp<kDppQuadXor1>(d);  // sum over the 16 lanes of the position
                d += dpp<kDppQuadXor2>(d);
                d += dpp<kDppRowRor4>(d);
                d += dpp<kDppRowRor8>(d);
                sr[it][hh] = p < p1 ? d * inv_sqrt_d : -INFINITY;
            }
        }
        float mn[G], rs[G];
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
            float v = sr[0][hh];
#pragma unroll
            for (int it = 1; it < kIt; ++it) v = fmaxf(v, sr[it][hh]);
            mn[hh] = fmaxf(m[hh], v);
            rs[hh] = m[hh] == -INFINITY ? 0.0f : expf(m[hh] - mn[hh]);
            m[hh] = mn[hh];
            l[hh] *= rs[hh];
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[hh][e] *= rs[hh];
        }
#pragma unroll
        for (int it = 0; it < kIt; ++it) {
            const int p = t0 + wave * 4 + pg + kStep * it;
            float v8[8];
            row_of(vraw[it], 1, p, v8);
#pragma unroll
            for (int hh = 0; hh < G; ++hh) {
                const float w = p < p1 ? expf(sr[it][hh] - m[hh]) : 0.0f;
                l[hh] += w;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[hh][e] = fmaf(w, v8[e], acc[hh][e]);
            }
        }
    };
    ASDSL_TIMELINE_STAMP(4, tl_wg, 2);
    for (int t = p0; t < p1; t += 2 * kTile) {  // uniform per workgroup
        if (t + kTile < p1) load_tile(t + kTile, kb, vb);
        process_tile(t, ka, va);
        if (t + kTile >= p1) break;
        if (t + 2 * kTile < p1) load_tile(t + 2 * kTile, ka, va);
        process_tile(t + kTile, kb, vb);
    }

    ASDSL_TIMELINE_STAMP(4, tl_wg, 3);
    merge_position_groups<G, kThreads>(m, l, acc, gml, gacc, ge,
                                       part + (static_cast<size_t>(kvh * G) * kMaxSplits + s) * kPartStride,
                                       static_cast<size_t>(kMaxSplits) * kPartStride);
    ASDSL_TIMELINE_STAMP(4, tl_wg, 4);
}

int attn_splits(int max_seq);

// Floats of the decode attention's work area: kMaxSplits partial rows per
// query head (every form; at most kMaxSplits splits whatever max_seq).
size_t attn_decode_work_floats(int n_heads, int max_seq) {
    (void)max_seq;
    return static_cast<size_t>(n_heads) * kMaxSplits * kPartStride;
}

// Merging in the attention kernel's last-arriving workgroup instead of the
// combine launch (device-coherent partial stores, an atomic count,
// device-coherent loads) measured slower: 13.2 us per layer at ctx 1024
// against 8.0 + 4.0.
// The kernel instance for G query heads per KV head (1..4) and the cache
// form: f(kernel) is called with the matching instantiation.
template <template <int, bool> class K, typename F>
asdsl_status with_attn_kernel(int G, bool q8, F&& f) {
    switch (G * 2 + (q8 ? 1 : 0)) {
        case 2: return f(K<1, false>::fn());
        case 3: return f(K<1, true>::fn());
        case 4: return f(K<2, false>::fn());
        case 5: return f(K<2, true>::fn());
        case 6: return f(K<3, false>::fn());
        case 7: return f(K<3, true>::fn());
        case 8: return f(K<4, false>::fn());
        case 9: return f(K<4, true>::fn());
        default:
            set_error("attention: n_heads / n_kv_heads must be 1..4");
            return ASDSL_ERR_UNSUPPORTED;
    }
}
template <int G, bool Q8>
struct DecodeAttnK {
    static auto fn() { return attn_decode_kernel<G, Q8, kShortForm.waves, kShortForm.tile / (4 * kShortForm.waves)>; }
};
template <int G, bool Q8>
struct DeepAttnK {
    static auto fn() { return attn_decode_kernel<G, Q8, kDeepForm.waves, kDeepForm.tile / (4 * kDeepForm.waves)>; }
};

// work: attn_decode_work_floats.  fold: the short form, partials at work
// (kMaxSplits rows per head) for the o_proj prologue; otherwise the long form
// and the combine kernel, att receiving the merged output.
asdsl_status launch_attention_decode(const float* qkv, const KvCache& kv, bool q8, const float* rc, const float* rs,
                                     const int* pos, float* att, float* work, int n_heads, int n_kv, int rot_half,
                                     int max_seq, int pos_limit, bool fold, uint32_t* flags, hipStream_t s) {
    const int limit = pos_limit < max_seq ? pos_limit : max_seq;
    const bool deep = !fold && limit > kDeepFrom;
    const FoldForm& f = fold ? kShortForm : deep ? kDeepForm : kLongForm;
    const dim3 grid(attn_max_splits(limit, f), n_kv);
    const dim3 block(f.waves * kWave);
    const int max_splits = f.max_splits;
    auto go = [&](auto kern) {
        return launch("attn_decode_kernel", kern, grid, block, 0, s, qkv, kv, rc, rs, pos, work, att, n_heads, n_kv,
                      max_seq, rot_half, max_splits, limit, flags);
    };
    const asdsl_status st = deep ? with_attn_kernel<DeepAttnK>(n_heads / n_kv, q8, go)
                                 : with_attn_kernel<DecodeAttnK>(n_heads / n_kv, q8, go);
    if (st != ASDSL_OK || fold) return st;
    const StageScope stage("attention_combine");
    return launch("attn_combine_kernel", attn_combine_kernel<0>, dim3(n_heads), dim3(combine_threads(grid.x)), 0, s,
                  static_cast<const float*>(work), pos, att, kMaxSplits, max_seq, limit, 0, 1, f.tile, f.max_splits,
                  static_cast<uint2*>(nullptr), static_cast<float2*>(nullptr), static_cast<float*>(nullptr));
}

int attn_splits(int max_seq) { return (max_seq + kSplit - 1) / kSplit; }

// Work buffer layout of one decode step (offsets in floats, 256-byte aligned).
struct DecodeWork {
    size_t hA, hB, qkv, att, o, gu, down, part, amax, flags, total;
};

size_t align64(size_t f) { return (f + 63) & ~static_cast<size_t>(63); }

DecodeWork decode_work(const asdsl_decode_model& m) {
    DecodeWork w{};
    size_t at = 0;
    auto take = [&](size_t n) {
        const size_t here = at;
        at += align64(n);
        return here;
    };
    const int qkv_dim = (m.n_heads + 2 * m.n_kv_heads) * m.head_dim;
    w.hA = take(m.hidden);
    w.hB = take(m.hidden);
    w.qkv = take(qkv_dim);
    w.att = take(static_cast<size_t>(m.n_heads) * m.head_dim);
    w.o = take(m.hidden);
    w.gu = take(2 * static_cast<size_t>(m.ffn));
    w.down = take(m.hidden);
    w.part = take(attn_decode_work_floats(m.n_heads, m.max_seq));
    w.amax = take(2);
    w.flags = take(1);  // ASDSL_DECODE_FLAG_* bits, set by the attention kernel, cleared by the host
    w.total = at;
    return w;
}

asdsl_status check_model(const asdsl_decode_model* m) {
    ASDSL_CHECK_ARG(m != nullptr, "decode: null model");
    ASDSL_CHECK_ARG(m->head_dim == kHeadDim, "decode: head_dim must be 128");
    ASDSL_CHECK_ARG(m->n_heads > 0 && m->n_kv_heads > 0 && m->n_heads % m->n_kv_heads == 0 &&
                        m->n_heads / m->n_kv_heads <= 4,
                    "decode: n_heads must be a multiple (1..4x) of n_kv_heads");
    ASDSL_CHECK_ARG(m->n_heads * m->head_dim == m->hidden, "decode: hidden must equal n_heads * head_dim");
    ASDSL_CHECK_ARG(m->rotary_dim > 0 && m->rotary_dim % 2 == 0 && m->rotary_dim <= m->head_dim,
                    "decode: rotary_dim must be even and <= head_dim");
    ASDSL_CHECK_ARG(m->hidden % 128 == 0 && m->ffn % 128 == 0 && m->hidden <= 8192 && m->ffn <= 8192,
                    "decode: hidden and ffn must be multiples of 128 and <= 8192");
    ASDSL_CHECK_ARG((m->gs_attn == 32 || m->gs_attn == 128) && (m->gs_ffn == 32 || m->gs_ffn == 128) &&
                        (m->gs_lm == 32 || m->gs_lm == 128),
                    "decode: group sizes must be 32 or 128");
    ASDSL_CHECK_ARG(m->n_layers > 0 && m->layers && m->embed && m->rms_out && m->lm_meta && m->lm_quant &&
                        m->rope_cos && m->rope_sin && m->vocab > 0 && m->max_seq > 0,
                    "decode: incomplete model description");
    ASDSL_CHECK_ARG(m->kv_format == ASDSL_KV_FP16 || m->kv_format == ASDSL_KV_INT8,
                    "decode: kv_format must be ASDSL_KV_FP16 or ASDSL_KV_INT8");
    for (int l = 0; l < m->n_layers; ++l) {
        const asdsl_decode_layer& L = m->layers[l];
        ASDSL_CHECK_ARG(L.k_cache && L.v_cache && reinterpret_cast<uintptr_t>(L.k_cache) % 16 == 0 &&
                            reinterpret_cast<uintptr_t>(L.v_cache) % 16 == 0,
                        "decode: layer %d: K/V caches must be non-null and 16-byte aligned", l);
        ASDSL_CHECK_ARG(m->kv_format != ASDSL_KV_INT8 || (L.k_scale && L.v_scale),
                        "decode: layer %d: the int8 cache needs its scale arrays", l);
    }
    return ASDSL_OK;
}


// ------------------------------------------------------------------ verify
// A multi-token pass over n tokens at positions pos .. pos + n - 1, the
// speculative verify of UnifiedEngine::forward_verify_batch
// (unified_engine.cpp:1774-1789): column c of every activation matrix is
// token c, the projections run as batched GEMVs (the dot4 form of
// asdsl_gemv_preq2_fused_batch, whose per-column arithmetic follows the
// single-column GEMV), and the elementwise steps use the decode step's
// formulas, so a column tracks the single-token step to fp32 rounding.
constexpr int kMaxVerifyTokens = 16;
constexpr int kNormThreads = 512;  // 8 waves, as the fused prologue of the norm-fed GEMVs

// H[c] = embed[tokens[c]] (fp16 -> fp32); clears the n argmax keys.
__global__ __launch_bounds__(256) void verify_embed_kernel(const uint16_t* __restrict__ embed,
                                                           const int* __restrict__ tokens, float* __restrict__ H,
                                                           int hidden, int vocab, unsigned long long* __restrict__ keys) {
    const int c = static_cast<int>(blockIdx.y);
    const int t0 = tokens[c];
    const int t = t0 >= 0 && t0 < vocab ? t0 : 0;
    const uint16_t* row = embed + static_cast<size_t>(t) * hidden;
    for (int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x); i < hidden;
         i += static_cast<int>(gridDim.x * blockDim.x))
        H[static_cast<size_t>(c) * hidden + i] = h2f(row[i]);
    if (blockIdx.x == 0 && threadIdx.x == 0) keys[c] = 0ull;
}

// Per column c (one workgroup): h = H[c] + D[c] (D may be null), written back
// to H[c]; X[c] = (h * inv_rms) * w with inv_rms = 1 / sqrt(sum(h^2)/K + eps)
// (residual_add_rmsnorm_f32, unified_engine.cpp:499-524).  The sum is formed
// in the order of the single-token GEMV's fused prologue at 8 waves (the plan
// of the norm-fed GEMVs at hidden 3072): thread t folds the 8-element chunks
// t, t + 512, ... element by element, then a xor butterfly per wave and the
// 8 wave sums in order, so both passes normalize identically.
// IMG_GS (32 or 128): X[c] is also quantized into the next batched GEMV's
// int8 image (image_store8, the values batch_quantize_kernel would form from
// X), and workgroups c >= ncols (the grid covers kImageCols columns) write
// that image's zero columns, so the GEMV needs no quantize launch of its own.
// inv_out (IMG_GS = 0 only): the single-token GEMV's factored form instead,
// X[c] = h * w and inv_out[c] = inv_rms, which the batched GEMV applies to
// its reduced rows (preq2_batch_exact), as the norm-fed GEMV's prologue and
// epilogue do.
template <int IMG_GS>
__global__ __launch_bounds__(kNormThreads) void verify_add_norm_kernel(float* __restrict__ H,
                                                                       const float* __restrict__ D,
                                                                       const float* __restrict__ w,
                                                                       float* __restrict__ X, int K, float eps,
                                                                       int ncols, uint2* __restrict__ img,
                                                                       float2* __restrict__ fac,
                                                                       float* __restrict__ us,
                                                                       float* __restrict__ inv_out) {
    __shared__ float red[kNormThreads / kWave];
    const int col = static_cast<int>(blockIdx.x);
    const int tid = static_cast<int>(threadIdx.x);
    const int nchunk = K >> 3;
    if constexpr (IMG_GS != 0) {
        if (col >= ncols) {
            const float z[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
            for (int base = 0; base < nchunk; base += kNormThreads)  // uniform per workgroup
                image_store8<IMG_GS>(z, base + tid, col, base + tid < nchunk, img, fac, us);
            return;
        }
    }
    const size_t c = static_cast<size_t>(col);
    float4* h = reinterpret_cast<float4*>(H + c * K);
    const float4* d = D ? reinterpret_cast<const float4*>(D + c * K) : nullptr;
    float4* x = reinterpret_cast<float4*>(X + c * K);
    const float4* w4 = reinterpret_cast<const float4*>(w);
    float ss = 0.0f;
    for (int ch = tid; ch < nchunk; ch += kNormThreads) {
        float v[8];
        const float4 a = h[2 * ch], b = h[2 * ch + 1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        if (d) {
            const float4 da = d[2 * ch], db = d[2 * ch + 1];
            v[0] += da.x; v[1] += da.y; v[2] += da.z; v[3] += da.w;
            v[4] += db.x; v[5] += db.y; v[6] += db.z; v[7] += db.w;
            h[2 * ch] = make_float4(v[0], v[1], v[2], v[3]);
            h[2 * ch + 1] = make_float4(v[4], v[5], v[6], v[7]);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, kWave);
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = ss;
    __syncthreads();
    float tot = red[0];
#pragma unroll
    for (int q = 1; q < kNormThreads / kWave; ++q) tot += red[q];
    const float inv_rms = 1.0f / sqrtf(tot / static_cast<float>(K) + eps);
    if (IMG_GS == 0 && inv_out) {
        if (tid == 0) inv_out[col] = inv_rms;
        for (int ch = tid; ch < nchunk; ch += kNormThreads) {
            const float4 a = h[2 * ch], b = h[2 * ch + 1];
            const float4 wa = w4[2 * ch], wb = w4[2 * ch + 1];
            x[2 * ch] = make_float4(a.x * wa.x, a.y * wa.y, a.z * wa.z, a.w * wa.w);
            x[2 * ch + 1] = make_float4(b.x * wb.x, b.y * wb.y, b.z * wb.z, b.w * wb.w);
        }
        return;
    }
    // the loop is uniform per workgroup (every lane of a quantization group
    // takes part); chunks past the end quantize a copy of the last chunk and
    // store nothing
    for (int base = 0; base < nchunk; base += kNormThreads) {
        const int ch = base + tid;
        const int cc = min(ch, nchunk - 1);
        const float4 a = h[2 * cc], b = h[2 * cc + 1];
        const float4 wa = w4[2 * cc], wb = w4[2 * cc + 1];
        const float v[8] = {(a.x * inv_rms) * wa.x, (a.y * inv_rms) * wa.y, (a.z * inv_rms) * wa.z,
                            (a.w * inv_rms) * wa.w, (b.x * inv_rms) * wb.x, (b.y * inv_rms) * wb.y,
                            (b.z * inv_rms) * wb.z, (b.w * inv_rms) * wb.w};
        if (ch < nchunk) {
            x[2 * ch] = make_float4(v[0], v[1], v[2], v[3]);
            x[2 * ch + 1] = make_float4(v[4], v[5], v[6], v[7]);
        }
        if constexpr (IMG_GS != 0) image_store8<IMG_GS>(v, ch, col, ch < nchunk, img, fac, us);
    }
}

// Dim d of a head row src rotated for position `pos` (rope_apply_inplace,
// unified_engine.cpp:499-540: pairs (i, i + rot_half) for i < rot_half, the
// rest passed through), fused as fmaf(x_i, c, -x_{i+h} * s).
__device__ __forceinline__ float rope_dim(const float* __restrict__ src, int d, int pos, int rot_half,
                                          const float* __restrict__ rope_cos, const float* __restrict__ rope_sin) {
    if (d >= 2 * rot_half) return src[d];
    const int i = d < rot_half ? d : d - rot_half;
    const float xf = src[i], xs = src[i + rot_half];
    const float cs = rope_cos[static_cast<size_t>(pos) * rot_half + i];
    const float sn = rope_sin[static_cast<size_t>(pos) * rot_half + i];
    return d < rot_half ? fmaf(xf, cs, -(xs * sn)) : fmaf(xf, sn, xs * cs);
}

// set_kv_cache's int8 rule (kv_q8_code) on a 64-dim block held 8 values a
// lane by the 8 lanes of an aligned group: codes to q[8], the scale returned.
__device__ __forceinline__ float kv_q8_codes8(const float (&x)[8], int (&q)[8]) {
    float a = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) a = fmaxf(a, fabsf(x[e]));
#pragma unroll
    for (int o = 4; o >= 1; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 8));
    const float scale = a > 1e-12f ? a * kInv127 : 1e-12f;
    const float inv = 1.0f / scale;
#pragma unroll
    for (int e = 0; e < 8; ++e) q[e] = static_cast<int>(fminf(fmaxf(__builtin_rintf(x[e] * inv), -127.0f), 127.0f));
    return scale;
}

// Dims 8*dc..+8 of a new row (fp32) in kv_load8's form: fp16 bits, or the 8
// codes and the block scale (the 8 lanes of the 64-dim block call together).
template <bool Q8>
__device__ __forceinline__ uint4 kv_pack8(const float (&x)[8]) {
    if constexpr (Q8) {
        int q[8];
        const float scale = kv_q8_codes8(x, q);
        uint32_t lo = 0u, hi = 0u;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            lo |= (static_cast<uint32_t>(q[e]) & 0xFFu) << (8 * e);
            hi |= (static_cast<uint32_t>(q[4 + e]) & 0xFFu) << (8 * e);
        }
        return make_uint4(lo, hi, __float_as_uint(scale), 0u);
    } else {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            w[e] = static_cast<uint32_t>(f2h(x[2 * e])) | (static_cast<uint32_t>(f2h(x[2 * e + 1])) << 16);
        return make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// Attention partials of column c (position pos + c) for one KV head and one
// split, with RoPE and the pass's own K/V rows done here: the column's G
// query heads are rotated from its qkv row; rows of positions at or past the
// pass's first (columns c' <= c) are rebuilt from column c''s qkv row
// exactly as the cache holds them (rotated key and value, rounded to fp16 or
// quantized to int8 codes and a scale per 64 dims), older rows come from the
// cache.  The workgroup whose split holds column c's own position stores
// that row into the cache; no other workgroup reads it there, so the pass
// needs no ordering between workgroups.  Columns past the cache do nothing.
template <int G, bool Q8>
__global__ __launch_bounds__(kAttnThreads) void verify_attn_partial_kernel(
    const float* __restrict__ QKV, KvCache kv, const float* __restrict__ rope_cos,
    const float* __restrict__ rope_sin, const int* __restrict__ pos_ptr, float* __restrict__ part, int n_heads,
    int n_kv, int max_seq, int nsplit, int rot_half) {
    __shared__ float q_s[G][kHeadDim];
    __shared__ float gml[kAttnThreads / 16][G][2];
    __shared__ __align__(16) float gacc[kAttnThreads / 16][G][kHeadDim];
    __shared__ float ge[G][kAttnThreads / 16];
    const int s = static_cast<int>(blockIdx.x);
    const int kvh = static_cast<int>(blockIdx.y);
    const int c = static_cast<int>(blockIdx.z);
    const int first = *pos_ptr;
    const int pos = first + c;
    const int p0 = s * kSplit;
    if (p0 > pos || pos < 0 || pos >= max_seq) return;
    const int p1 = min(p0 + kSplit, pos + 1);
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & (kWave - 1);
    const int wave = tid >> 6;
    const int pg = lane >> 4;
    const int dc = lane & 15;
    const size_t row0 = static_cast<size_t>(kvh) * max_seq;
    const size_t qkv_row = static_cast<size_t>(n_heads + 2 * n_kv) * kHeadDim;
    constexpr int kIt = kSplit / 16;
    uint4 kraw[kIt], vraw[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
        const int p = p0 + wave * 4 + pg + 16 * it;  // uniform over the 16 lanes of a position
        if (p < p1 && p < first) {
            kraw[it] = kv_load8<Q8>(kv.k, kv.ks, row0 + p, dc);
            vraw[it] = kv_load8<Q8>(kv.v, kv.vs, row0 + p, dc);
        } else if (p < p1) {
            const float* row = QKV + static_cast<size_t>(p - first) * qkv_row;
            const float* ksrc = row + static_cast<size_t>(n_heads + kvh) * kHeadDim;
            const float* vsrc = row + static_cast<size_t>(n_heads + n_kv + kvh) * kHeadDim;
            float k8[8], v8[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                k8[e] = rope_dim(ksrc, 8 * dc + e, p, rot_half, rope_cos, rope_sin);
                v8[e] = vsrc[8 * dc + e];
            }
            kraw[it] = kv_pack8<Q8>(k8);
            vraw[it] = kv_pack8<Q8>(v8);
            if (p == pos) {  // this column's own row: into the cache
                const size_t crow = row0 + p;
                if constexpr (Q8) {
                    *reinterpret_cast<uint2*>(static_cast<int8_t*>(kv.k) + crow * kHeadDim + 8 * dc) =
                        make_uint2(kraw[it].x, kraw[it].y);
                    *reinterpret_cast<uint2*>(static_cast<int8_t*>(kv.v) + crow * kHeadDim + 8 * dc) =
                        make_uint2(vraw[it].x, vraw[it].y);
                    if ((dc & 7) == 0) {
                        kv.ks[crow * 2 + (dc >> 3)] = __uint_as_float(kraw[it].z);
                        kv.vs[crow * 2 + (dc >> 3)] = __uint_as_float(vraw[it].z);
                    }
                } else {
                    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(kv.k) + crow * kHeadDim + 8 * dc) = kraw[it];
                    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(kv.v) + crow * kHeadDim + 8 * dc) = vraw[it];
                }
            }
        } else {
            kraw[it] = make_uint4(0u, 0u, 0u, 0u);
            vraw[it] = kraw[it];
        }
    }
    const float* qsrc = QKV + static_cast<size_t>(c) * qkv_row + static_cast<size_t>(kvh * G) * kHeadDim;
    for (int e = tid; e < G * kHeadDim; e += kAttnThreads)
        q_s[e / kHeadDim][e % kHeadDim] = rope_dim(qsrc + (e / kHeadDim) * kHeadDim, e % kHeadDim, pos, rot_half,
                                                   rope_cos, rope_sin);
    __syncthreads();
    float qr[G][8];
#pragma unroll
    for (int hh = 0; hh < G; ++hh)
#pragma unroll
        for (int e = 0; e < 8; ++e) qr[hh][e] = q_s[hh][8 * dc + e];
    attn_split_core<G, false, Q8>(kraw, vraw, qr, p0, p1, pos, nullptr, gml, gacc, ge,
                              part + ((static_cast<size_t>(c) * n_heads + kvh * G) * nsplit + s) * kPartStride,
                              static_cast<size_t>(nsplit) * kPartStride);
}

// S[c] = SwiGLU(gate, up) of GU[c] = [gate | up] with the FATReLU threshold
// (swiglu_inplace, unified_engine.cpp:803-857; the decode prologue's formula).
// S[c] = swiglu(GU[c][0:ffn], GU[c][ffn:2ffn]), one 8-element chunk per
// thread (grid: ceil(ffn / 2048) x columns).  IMG_GS: also the down GEMV's
// int8 image of S (image_store8), with zero image columns for c >= ncols (the
// grid then covers kImageCols columns).
template <int IMG_GS>
__global__ __launch_bounds__(256) void verify_swiglu_kernel(const float* __restrict__ GU, float* __restrict__ S,
                                                            int ffn, float thr, int ncols, uint2* __restrict__ img,
                                                            float2* __restrict__ fac, float* __restrict__ us) {
    const int col = static_cast<int>(blockIdx.y);
    const size_t c = static_cast<size_t>(col);
    const int nchunk = ffn >> 3;
    const int ch = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
    const int cc = min(ch, nchunk - 1);
    float v[8];
    if (IMG_GS != 0 && col >= ncols) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.0f;
    } else {
        const float* g = GU + c * 2 * ffn + 8 * cc;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = swiglu_ref(g[e], g[ffn + e], thr);
        if (ch < nchunk) {
            float4* sp = reinterpret_cast<float4*>(S + c * ffn + 8 * ch);
            sp[0] = make_float4(v[0], v[1], v[2], v[3]);
            sp[1] = make_float4(v[4], v[5], v[6], v[7]);
        }
    }
    if constexpr (IMG_GS != 0) image_store8<IMG_GS>(v, ch, col, ch < nchunk, img, fac, us);
}

// keys[c] = max over rows of argmax_key(logits[c][row], row): the largest
// logit, the first row among equals (argmax_f32_avx2, unified_engine.cpp:207-233).
// A thread takes kArgmaxRows rows 256 apart per step, all loaded before any
// is compared.  kArgmaxWgs workgroups per column: each ends in one atomicMax
// on the column's key, and those serialize (196 per key measured 30 us
// against 12 for 64).
constexpr int kArgmaxRows = 8;
constexpr int kArgmaxWgs = 64;
__global__ __launch_bounds__(256) void verify_argmax_kernel(const float* __restrict__ logits, int vocab,
                                                            unsigned long long* __restrict__ keys) {
    __shared__ unsigned long long red[256 / kWave];
    const size_t c = blockIdx.y;
    unsigned long long best = 0ull;
    for (int r0 = static_cast<int>(blockIdx.x * blockDim.x * kArgmaxRows + threadIdx.x); r0 < vocab;
         r0 += static_cast<int>(gridDim.x * blockDim.x * kArgmaxRows)) {
        float v[kArgmaxRows];
#pragma unroll
        for (int j = 0; j < kArgmaxRows; ++j) {
            const int r = r0 + j * static_cast<int>(blockDim.x);
            v[j] = logits[c * vocab + (r < vocab ? r : r0)];  // past the vocabulary: row r0 again
        }
#pragma unroll
        for (int j = 0; j < kArgmaxRows; ++j) {
            const int r = r0 + j * static_cast<int>(blockDim.x);
            const unsigned long long k = r < vocab ? argmax_key(v[j], r) : 0ull;
            best = k > best ? k : best;
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const unsigned long long other = __shfl_xor(best, o, kWave);
        best = other > best ? other : best;
    }
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long tot = red[0];
#pragma unroll
        for (int q = 1; q < 256 / kWave; ++q) tot = red[q] > tot ? red[q] : tot;
        atomicMax(keys + c, tot);
    }
}

__global__ void verify_tokens_kernel(const unsigned long long* __restrict__ keys, int* __restrict__ next, int n) {
    const int c = static_cast<int>(threadIdx.x);
    if (c < n) next[c] = static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(keys[c]));
}

// Zero the cache rows [from, max_seq) of every KV head (zero_kv_from,
// unified_engine.cpp:1263-1283), 16-byte stores.
__global__ __launch_bounds__(256) void kv_zero_kernel(uint4* __restrict__ k, uint4* __restrict__ v, int n_kv,
                                                      int max_seq, int from) {
    const size_t per_head = static_cast<size_t>(max_seq - from) * (kHeadDim / 8);
    const size_t total = per_head * n_kv;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const size_t h = i / per_head;
        const size_t at = (h * max_seq + from) * (kHeadDim / 8) + (i - h * per_head);
        k[at] = make_uint4(0u, 0u, 0u, 0u);
        v[at] = make_uint4(0u, 0u, 0u, 0u);
    }
}

// The int8 cache's rows [from, max_seq): codes 0 and scales 1.0, as
// zero_kv_from leaves them (unified_engine.cpp:1263-1283).
__global__ __launch_bounds__(256) void kv_zero_q8_kernel(uint4* __restrict__ k, uint4* __restrict__ v,
                                                         float* __restrict__ ks, float* __restrict__ vs, int n_kv,
                                                         int max_seq, int from) {
    constexpr int kU = kHeadDim / 16;  // 16-byte units per row
    const size_t rows = static_cast<size_t>(max_seq - from);
    const size_t total = rows * n_kv * kU;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const size_t h = i / (rows * kU);
        const size_t r = (i - h * rows * kU) / kU;
        const size_t u = i % kU;
        const size_t crow = h * max_seq + from + r;
        k[crow * kU + u] = make_uint4(0u, 0u, 0u, 0u);
        v[crow * kU + u] = make_uint4(0u, 0u, 0u, 0u);
        if (u < 2) {
            ks[crow * 2 + u] = 1.0f;
            vs[crow * 2 + u] = 1.0f;
        }
    }
}

template <int G, bool Q8>
struct VerifyAttnK {
    static auto fn() { return verify_attn_partial_kernel<G, Q8>; }
};

// Work buffer layout of a verify pass of up to n tokens (offsets in floats).
struct VerifyWork {
    size_t H, X, QKV, part, att, O, GU, S, keys, inv, mimg, mimg_bytes, total;
};

VerifyWork verify_work(const asdsl_decode_model& m, int n) {
    VerifyWork w{};
    size_t at = 0;
    auto take = [&](size_t cnt) {
        const size_t here = at;
        at += align64(cnt);
        return here;
    };
    const size_t N = static_cast<size_t>(n);
    const int qkv_dim = (m.n_heads + 2 * m.n_kv_heads) * m.head_dim;
    w.H = take(N * m.hidden);
    w.X = take(N * (m.hidden > m.ffn ? m.hidden : m.ffn));
    w.QKV = take(N * qkv_dim);
    w.part = take(N * m.n_heads * attn_splits(m.max_seq) * kPartStride);
    w.att = take(N * m.n_heads * m.head_dim);
    w.O = take(N * m.hidden);
    w.GU = take(N * 2 * m.ffn);
    w.S = take(N * m.ffn);
    w.keys = take(2 * N);
    w.inv = take(N);
    // the MFMA batched GEMV's column image (the widest input, K = max(hidden, ffn))
    w.mimg_bytes = asdsl_gemv_preq2_fused_batch_work_bytes(m.hidden > m.ffn ? m.hidden : m.ffn);
    w.mimg = take((w.mimg_bytes + sizeof(float) - 1) / sizeof(float));
    w.total = at;
    return w;
}

}  // namespace
}  // namespace asdsl

using namespace asdsl;

extern "C" asdsl_status asdsl_gemv_preq2_fused(const uint8_t* meta, const uint8_t* quant, const float* x, float* y,
                                               int out_features, int in_features, int group_size,
                                               asdsl_stream_t stream);
extern "C" asdsl_status asdsl_gemv_preq2_rmsnorm(const uint8_t* meta, const uint8_t* quant, const float* h_in,
                                                 const float* delta, const float* norm_w, float* h_out, float* y,
                                                 int out_features, int in_features, int group_size, float eps,
                                                 unsigned long long* argmax_key, asdsl_stream_t stream);
extern "C" asdsl_status asdsl_gemv_preq2_swiglu(const uint8_t* meta, const uint8_t* quant, const float* gate_up,
                                                float* y, int out_features, int in_features, int group_size,
                                                float threshold, asdsl_stream_t stream);
extern "C" asdsl_status asdsl_gemv_preq2_rmsnorm_swiglu(const uint8_t* meta, const uint8_t* quant, const float* h_in,
                                                        const float* delta, const float* norm_w, float* h_out,
                                                        float* s_out, int ffn, int in_features, int group_size,
                                                        float eps, float threshold, asdsl_stream_t stream);

extern "C" size_t asdsl_attention_work_floats(int n_heads, int max_seq) {
    return n_heads > 0 && max_seq > 0 ? attn_decode_work_floats(n_heads, max_seq) : 0;
}

namespace {
asdsl_status check_attention_args(const char* what, const void* qkv, const void* k_cache, const void* v_cache,
                                  const void* rope_cos, const void* rope_sin, const void* pos, const void* att_out,
                                  const void* work, int n_heads, int n_kv_heads, int head_dim, int rotary_dim,
                                  int max_seq) {
    ASDSL_CHECK_ARG(qkv && k_cache && v_cache && rope_cos && rope_sin && pos && att_out && work,
                    "%s: null pointer", what);
    ASDSL_CHECK_ARG(head_dim == kHeadDim, "%s: head_dim must be 128", what);
    ASDSL_CHECK_ARG(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0 && n_heads / n_kv_heads <= 4,
                    "%s: n_heads must be a multiple (1..4x) of n_kv_heads", what);
    ASDSL_CHECK_ARG(rotary_dim > 0 && rotary_dim % 2 == 0 && rotary_dim <= head_dim,
                    "%s: rotary_dim must be even and <= head_dim", what);
    ASDSL_CHECK_ARG(max_seq > 0, "%s: max_seq must be positive", what);
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(k_cache) % 16 == 0 && reinterpret_cast<uintptr_t>(v_cache) % 16 == 0,
                    "%s: caches must be 16-byte aligned", what);
    return ASDSL_OK;
}
}  // namespace

extern "C" asdsl_status asdsl_attention_f16kv(const float* qkv, uint16_t* k_cache, uint16_t* v_cache,
                                              const float* rope_cos, const float* rope_sin, const int* pos,
                                              float* att_out, float* work, int n_heads, int n_kv_heads,
                                              int head_dim, int rotary_dim, int max_seq, asdsl_stream_t stream) {
    const asdsl_status cs = check_attention_args("attention_f16kv", qkv, k_cache, v_cache, rope_cos, rope_sin, pos,
                                                 att_out, work, n_heads, n_kv_heads, head_dim, rotary_dim, max_seq);
    if (cs != ASDSL_OK) return cs;
    const KvCache kv{k_cache, v_cache, nullptr, nullptr};
    return launch_attention_decode(qkv, kv, false, rope_cos, rope_sin, pos, att_out, work, n_heads, n_kv_heads,
                                   rotary_dim / 2, max_seq, max_seq, false, nullptr, as_hip(stream));
}

extern "C" asdsl_status asdsl_attention_q8kv(const float* qkv, int8_t* k_cache, int8_t* v_cache, float* k_scale,
                                             float* v_scale, const float* rope_cos, const float* rope_sin,
                                             const int* pos, float* att_out, float* work, int n_heads, int n_kv_heads,
                                             int head_dim, int rotary_dim, int max_seq, asdsl_stream_t stream) {
    const asdsl_status cs = check_attention_args("attention_q8kv", qkv, k_cache, v_cache, rope_cos, rope_sin, pos,
                                                 att_out, work, n_heads, n_kv_heads, head_dim, rotary_dim, max_seq);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(k_scale && v_scale, "attention_q8kv: null scale array");
    const KvCache kv{k_cache, v_cache, k_scale, v_scale};
    return launch_attention_decode(qkv, kv, true, rope_cos, rope_sin, pos, att_out, work, n_heads, n_kv_heads,
                                   rotary_dim / 2, max_seq, max_seq, false, nullptr, as_hip(stream));
}

extern "C" size_t asdsl_decode_work_bytes(const asdsl_decode_model* model) {
    if (check_model(model) != ASDSL_OK) return 0;
    return decode_work(*model).total * sizeof(float);
}

extern "C" size_t asdsl_decode_flags_offset(const asdsl_decode_model* model) {
    if (check_model(model) != ASDSL_OK) return 0;
    return decode_work(*model).flags * sizeof(float);
}

extern "C" asdsl_status asdsl_decode_token_upto(const asdsl_decode_model* model, int* token, int* pos, int pos_limit,
                                                float* logits, void* work, asdsl_stream_t stream) {
    const asdsl_status cs = check_model(model);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(token && pos && logits && work, "decode_token: null pointer");
    ASDSL_CHECK_ARG(pos_limit > 0, "decode_token: pos_limit must be positive");
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(work) % 256 == 0, "decode_token: work must be 256-byte aligned");
    const asdsl_decode_model& m = *model;
    const DecodeWork w = decode_work(m);
    float* base = static_cast<float*>(work);
    float* hA = base + w.hA;
    float* hB = base + w.hB;
    float* qkv = base + w.qkv;
    float* att = base + w.att;
    float* o = base + w.o;
    float* gu = base + w.gu;
    float* down = base + w.down;
    float* part = base + w.part;
    auto* amax = reinterpret_cast<unsigned long long*>(base + w.amax);
    auto* flags = reinterpret_cast<uint32_t*>(base + w.flags);
    hipStream_t s = as_hip(stream);
    const int qkv_dim = (m.n_heads + 2 * m.n_kv_heads) * m.head_dim;
    const int q_dim = m.n_heads * m.head_dim;
    // The attention form follows pos_limit (attn_fold): below 512 o_proj's
    // prologue merges the splits, from there the combine kernel does.
    // ASDSL_HIP_NO_COMBINE_FOLD=1 always takes the combine kernel.
    static const int no_fold = env_knob("ASDSL_HIP_NO_COMBINE_FOLD");
    const int limit = pos_limit < m.max_seq ? pos_limit : m.max_seq;
    const bool fold = no_fold == 0 && attn_fold(limit);
    const FoldForm& form = kShortForm;  // o_proj's prologue merge (fold only)
    const bool q8 = m.kv_format == ASDSL_KV_INT8;

    // Layer 0's qkv GEMV reads the embedding row itself (and stores it to hA,
    // clearing the argmax key) when the table is 16-byte aligned; otherwise
    // embed_kernel does that first.
    const bool embed_fold = reinterpret_cast<uintptr_t>(m.embed) % 16 == 0;
    asdsl_status st = ASDSL_OK;
    if (!embed_fold) {
        const StageScope stage("embed");
        st = launch("embed_kernel", embed_kernel, dim3((m.hidden + 1023) / 1024), dim3(256), 0, s, m.embed,
                    static_cast<const int*>(token), hA, m.hidden, m.vocab, amax);
        if (st != ASDSL_OK) return st;
    }
    // The residual stream enters layer l in `cur`; layer l > 0 adds the
    // previous down output in its qkv prologue and writes the sum to `nxt`.
    float* cur = hA;
    float* nxt = hB;
    for (int l = 0; l < m.n_layers; ++l) {
        const asdsl_decode_layer& L = m.layers[l];
        StageScope stage("qkv");
        if (l > 0) {
            st = asdsl_gemv_preq2_rmsnorm(L.qkv_meta, L.qkv_quant, cur, down, L.rms_att, nxt, qkv, qkv_dim,
                                          m.hidden, m.gs_attn, m.rms_eps, nullptr, stream);
            std::swap(cur, nxt);
        } else if (embed_fold) {
            st = preq2_embed_rmsnorm(L.qkv_meta, L.qkv_quant, m.embed, static_cast<const int*>(token), m.vocab,
                                     L.rms_att, hA, qkv, qkv_dim, m.hidden, m.gs_attn, m.rms_eps, amax, stream);
        } else {
            st = asdsl_gemv_preq2_rmsnorm(L.qkv_meta, L.qkv_quant, cur, nullptr, L.rms_att, nullptr, qkv, qkv_dim,
                                          m.hidden, m.gs_attn, m.rms_eps, nullptr, stream);
        }
        if (st != ASDSL_OK) return st;
        const KvCache kv{L.k_cache, L.v_cache, L.k_scale, L.v_scale};
        g_stage = "attention";  // the combine labels itself
        st = launch_attention_decode(qkv, kv, q8, m.rope_cos, m.rope_sin, pos, att, part, m.n_heads,
                                     m.n_kv_heads, m.rotary_dim / 2, m.max_seq, limit, fold, flags, s);
        if (st != ASDSL_OK) return st;
        g_stage = "o_proj";
        st = fold ? preq2_fused_combine(L.o_meta, L.o_quant, att, o, m.hidden, q_dim, m.gs_attn, part, pos, kMaxSplits,
                                        form.tile, form.max_splits, kPartStride, kHeadDim, m.max_seq, limit, stream)
                  : asdsl_gemv_preq2_fused(L.o_meta, L.o_quant, att, o, m.hidden, q_dim, m.gs_attn, stream);
        if (st != ASDSL_OK) return st;
        // gate_up with SwiGLU in its epilogue (gate and up rows in one
        // workgroup), down on the result; the SwiGLU prologue form otherwise
        g_stage = "gate_up";
        st = asdsl_gemv_preq2_rmsnorm_swiglu(L.gu_meta, L.gu_quant, cur, o, L.rms_ffn, nxt, gu, m.ffn, m.hidden,
                                             m.gs_ffn, m.rms_eps, L.fatrelu_threshold, stream);
        if (st == ASDSL_OK) {
            std::swap(cur, nxt);
            g_stage = "down";
            st = asdsl_gemv_preq2_fused(L.down_meta, L.down_quant, gu, down, m.hidden, m.ffn, m.gs_ffn, stream);
        } else if (st == ASDSL_ERR_UNSUPPORTED) {
            st = asdsl_gemv_preq2_rmsnorm(L.gu_meta, L.gu_quant, cur, o, L.rms_ffn, nxt, gu, 2 * m.ffn, m.hidden,
                                          m.gs_ffn, m.rms_eps, nullptr, stream);
            if (st != ASDSL_OK) return st;
            std::swap(cur, nxt);
            g_stage = "down";
            st = asdsl_gemv_preq2_swiglu(L.down_meta, L.down_quant, gu, down, m.hidden, m.ffn, m.gs_ffn,
                                         L.fatrelu_threshold, stream);
        }
        if (st != ASDSL_OK) return st;
    }
    StageScope stage("lm_head");
    st = asdsl_gemv_preq2_rmsnorm(m.lm_meta, m.lm_quant, cur, down, m.rms_out, nullptr, logits, m.vocab, m.hidden,
                                  m.gs_lm, m.rms_eps, amax, stream);
    if (st != ASDSL_OK) return st;
    g_stage = "finalize";
    return launch("finalize_kernel", finalize_kernel, dim3(1), dim3(64), 0, s,
                  static_cast<const unsigned long long*>(amax), token, pos);
}

extern "C" asdsl_status asdsl_decode_token(const asdsl_decode_model* model, int* token, int* pos, float* logits,
                                           void* work, asdsl_stream_t stream) {
    return asdsl_decode_token_upto(model, token, pos, model ? model->max_seq : 1, logits, work, stream);
}

extern "C" size_t asdsl_decode_verify_work_bytes(const asdsl_decode_model* model, int max_tokens) {
    if (check_model(model) != ASDSL_OK || max_tokens < 1 || max_tokens > kMaxVerifyTokens) return 0;
    return verify_work(*model, max_tokens).total * sizeof(float);
}

extern "C" asdsl_status asdsl_decode_verify(const asdsl_decode_model* model, const int* tokens, int n_tokens,
                                            const int* pos, float* logits, int* next_tokens, void* work,
                                            asdsl_stream_t stream) {
    const asdsl_status cs = check_model(model);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(tokens && pos && logits && next_tokens && work, "decode_verify: null pointer");
    ASDSL_CHECK_ARG(n_tokens >= 1 && n_tokens <= kMaxVerifyTokens, "decode_verify: n_tokens must be in [1, %d]",
                    kMaxVerifyTokens);
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(work) % 256 == 0, "decode_verify: work must be 256-byte aligned");
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(logits) % 16 == 0, "decode_verify: logits must be 16-byte aligned");
    const asdsl_decode_model& m = *model;
    const int n = n_tokens;
    const VerifyWork w = verify_work(m, n);
    float* base = static_cast<float*>(work);
    float* H = base + w.H;
    float* X = base + w.X;
    float* QKV = base + w.QKV;
    float* part = base + w.part;
    float* att = base + w.att;
    float* O = base + w.O;
    float* GU = base + w.GU;
    float* S = base + w.S;
    auto* keys = reinterpret_cast<unsigned long long*>(base + w.keys);
    float* INV = base + w.inv;
    void* mimg = base + w.mimg;
    hipStream_t s = as_hip(stream);
    const int qkv_dim = (m.n_heads + 2 * m.n_kv_heads) * m.head_dim;
    const int q_dim = m.n_heads * m.head_dim;
    const int nsplit = attn_splits(m.max_seq);
    const int G = m.n_heads / m.n_kv_heads;
    const bool q8 = m.kv_format == ASDSL_KV_INT8;
    // Every projection repeats the single-token GEMV's arithmetic on each
    // column, and the norm-fed ones its norm form (the normed input, or with
    // ASDSL_HIP_NORM_FACTORED h * w quantized and 1/rms applied to the
    // reduced rows): below 2048 positions, where the attention splits
    // coincide too, every column then gives the single-token step's logits,
    // K/V rows and token bit for bit, as lossless speculative decoding needs.
    // From 4 columns (ASDSL_HIP_VERIFY_EXACT_MFMA_MIN_N, read per call), where
    // the single-token shape allows (preq2_batch_exact_mfma_applies), the
    // projection is the exact MFMA form on an activation image that the
    // kernel before it writes (the norm, the combine, the SwiGLU): the weights
    // stream once for up to 16 columns (32-layer pass at ctx 1024, against
    // the dot4 form: 1.94 against 1.97 ms at 4 columns, 1.95 against 2.18 at
    // 5, 2.06 against 2.70 at 8, 2.29 against 4.73 at 16; at 2 and 3 columns
    // dot4 is faster, 1.53 against 1.89 and 1.79 against 1.90).  Otherwise, with the
    // factored norm or ASDSL_HIP_VERIFY_DOT4=1 (read per call), the dot4
    // batched GEMV in the single-token launch shape (preq2_batch_exact).
    // ASDSL_HIP_VERIFY_MFMA=1 (read per call) takes the MFMA batched GEMV in
    // its own order instead: a column's int8 activations can then round
    // differently from the single-token step's.
    const bool mfma = env_knob("ASDSL_HIP_VERIFY_MFMA") > 0;
    const bool factored_norm = !mfma && preq2_norm_factored();
    const int exact_min_n = env_knob("ASDSL_HIP_VERIFY_EXACT_MFMA_MIN_N");
    const bool exact_mfma = !mfma && !factored_norm && env_knob("ASDSL_HIP_VERIFY_DOT4") == 0 &&
                            n >= (exact_min_n > 0 ? exact_min_n : 4);
    // dot4 in the single-token launch shape, else (a shape whose split masks
    // units) the batched GEMV's own dot4 plan
    auto gemv_exact = [&](const uint8_t* meta, const uint8_t* quant, const float* Xin, const float* inv, float* Y,
                          int M, int K, int gs) -> asdsl_status {
        const asdsl_status r = preq2_batch_exact(meta, quant, Xin, inv, Y, M, K, gs, n, stream);
        if (r != ASDSL_ERR_UNSUPPORTED || inv) return r;
        return preq2_fused_batch(meta, quant, Xin, Y, M, K, gs, n, stream, false, mimg, w.mimg_bytes);
    };

    asdsl_status st = launch("verify_embed_kernel", verify_embed_kernel, dim3((m.hidden + 1023) / 1024, n), dim3(256),
                             0, s, m.embed, tokens, H, m.hidden, m.vocab, keys);
    if (st != ASDSL_OK) return st;
    // The norm, combine and SwiGLU kernels write the next projection's int8
    // image themselves when that projection takes an image-fed form (1: the
    // MFMA form, 2: the exact MFMA form), which then runs without a quantize
    // launch of its own.
    auto* img = static_cast<uint2*>(mimg);
    auto fac_of = [&](int K) { return reinterpret_cast<float2*>(static_cast<uint8_t*>(mimg) + image_fac_offset(K)); };
    auto us_of = [&](int K) { return reinterpret_cast<float*>(static_cast<uint8_t*>(mimg) + image_us_offset(K)); };
    auto image_form = [&](const uint8_t* meta, const uint8_t* quant, int M, int K, int gs) -> int {
        if (mfma) return preq2_batch_image_applies(meta, quant, M, K, gs, n, true) ? 1 : 0;
        return exact_mfma && preq2_batch_exact_mfma_applies(M, K, gs, n) ? 2 : 0;
    };
    auto image_gemv = [&](int form, const uint8_t* meta, const uint8_t* quant, float* Y, int M, int K,
                          int gs) -> asdsl_status {
        return form == 1 ? preq2_batch_mfma_image(meta, quant, mimg, Y, M, K, gs, n, stream)
                         : preq2_batch_exact_mfma_image(meta, quant, mimg, Y, M, K, gs, n, stream);
    };
    auto norm_then_gemv = [&](const float* D, const float* nw, const uint8_t* meta, const uint8_t* quant, float* Y,
                              int M, int gs) -> asdsl_status {
        const int K = m.hidden;
        const int form = image_form(meta, quant, M, K, gs);
        if (form != 0) {
            asdsl_status r = launch("verify_add_norm_kernel",
                                    gs == 32 ? verify_add_norm_kernel<32> : verify_add_norm_kernel<128>,
                                    dim3(kImageCols), dim3(kNormThreads), 0, s, H, D, nw, X, K, m.rms_eps, n, img,
                                    fac_of(K), us_of(K), static_cast<float*>(nullptr));
            if (r != ASDSL_OK) return r;
            return image_gemv(form, meta, quant, Y, M, K, gs);
        }
        // the single-token GEMVs' norm form: the reference's order (normed
        // X, below) or the factored one; the factored form's 1/rms sum
        // follows the 8-wave prologue of the norm-fed GEMVs, which covers
        // K <= 4096 (the only plan they take there)
        const bool factored = factored_norm && K <= 4096 && K % 8 == 0;
        asdsl_status r = launch("verify_add_norm_kernel", verify_add_norm_kernel<0>, dim3(n), dim3(kNormThreads), 0, s,
                                H, D, nw, X, K, m.rms_eps, n, static_cast<uint2*>(nullptr),
                                static_cast<float2*>(nullptr), static_cast<float*>(nullptr), factored ? INV : nullptr);
        if (r != ASDSL_OK) return r;
        if (factored) {
            r = preq2_batch_exact(meta, quant, X, INV, Y, M, K, gs, n, stream);
            if (r != ASDSL_ERR_UNSUPPORTED) return r;
            // no exact shape: normalize in place and take the plain batched form
            r = launch("verify_add_norm_kernel", verify_add_norm_kernel<0>, dim3(n), dim3(kNormThreads), 0, s, H,
                       static_cast<const float*>(nullptr), nw, X, K, m.rms_eps, n, static_cast<uint2*>(nullptr),
                       static_cast<float2*>(nullptr), static_cast<float*>(nullptr), static_cast<float*>(nullptr));
            if (r != ASDSL_OK) return r;
        }
        return mfma ? preq2_fused_batch(meta, quant, X, Y, M, K, gs, n, stream, true, mimg, w.mimg_bytes)
                    : gemv_exact(meta, quant, X, nullptr, Y, M, K, gs);
    };
    // H carries the residual stream of every column; O (attention output
    // projection) and S -> O (down projection) are added in by the next norm.
    const float* pending = nullptr;
    for (int l = 0; l < m.n_layers; ++l) {
        const asdsl_decode_layer& L = m.layers[l];
        st = norm_then_gemv(pending, L.rms_att, L.qkv_meta, L.qkv_quant, QKV, qkv_dim, m.gs_attn);
        if (st != ASDSL_OK) return st;
        const KvCache kv{L.k_cache, L.v_cache, L.k_scale, L.v_scale};
        const dim3 pgrid(nsplit, m.n_kv_heads, n);
        st = with_attn_kernel<VerifyAttnK>(G, q8, [&](auto kern) {
            return launch("verify_attn_partial_kernel", kern, pgrid, dim3(kAttnThreads), 0, s,
                          static_cast<const float*>(QKV), kv, m.rope_cos, m.rope_sin, pos, part, m.n_heads,
                          m.n_kv_heads, m.max_seq, nsplit, m.rotary_dim / 2);
        });
        if (st != ASDSL_OK) return st;
        const int o_form = image_form(L.o_meta, L.o_quant, m.hidden, q_dim, m.gs_attn);
        if (o_form != 0) {
            st = launch("attn_combine_kernel", m.gs_attn == 32 ? attn_combine_kernel<32> : attn_combine_kernel<128>,
                        dim3(m.n_heads, kImageCols), dim3(combine_threads(nsplit)), 0, s, static_cast<const float*>(part), pos,
                        att, nsplit, m.max_seq, m.max_seq, 0, n, 0, 0, img, fac_of(q_dim), us_of(q_dim));
            if (st != ASDSL_OK) return st;
            st = image_gemv(o_form, L.o_meta, L.o_quant, O, m.hidden, q_dim, m.gs_attn);
        } else {
            st = launch("attn_combine_kernel", attn_combine_kernel<0>, dim3(m.n_heads, n), dim3(combine_threads(nsplit)), 0, s,
                        static_cast<const float*>(part), pos, att, nsplit, m.max_seq, m.max_seq, 0, n, 0, 0,
                        static_cast<uint2*>(nullptr), static_cast<float2*>(nullptr), static_cast<float*>(nullptr));
            if (st != ASDSL_OK) return st;
            st = mfma ? preq2_fused_batch(L.o_meta, L.o_quant, att, O, m.hidden, q_dim, m.gs_attn, n, stream, true,
                                          mimg, w.mimg_bytes)
                      : gemv_exact(L.o_meta, L.o_quant, att, nullptr, O, m.hidden, q_dim, m.gs_attn);
        }
        if (st != ASDSL_OK) return st;
        st = norm_then_gemv(O, L.rms_ffn, L.gu_meta, L.gu_quant, GU, 2 * m.ffn, m.gs_ffn);
        if (st != ASDSL_OK) return st;
        const int down_form = image_form(L.down_meta, L.down_quant, m.hidden, m.ffn, m.gs_ffn);
        const int sw_chunks = (m.ffn / 8 + 255) / 256;
        if (down_form != 0) {
            st = launch("verify_swiglu_kernel", m.gs_ffn == 32 ? verify_swiglu_kernel<32> : verify_swiglu_kernel<128>,
                        dim3(sw_chunks, kImageCols), dim3(256), 0, s, static_cast<const float*>(GU), S, m.ffn,
                        L.fatrelu_threshold, n, img, fac_of(m.ffn), us_of(m.ffn));
            if (st != ASDSL_OK) return st;
            st = image_gemv(down_form, L.down_meta, L.down_quant, O, m.hidden, m.ffn, m.gs_ffn);
        } else {
            st = launch("verify_swiglu_kernel", verify_swiglu_kernel<0>, dim3(sw_chunks, n), dim3(256), 0, s,
                        static_cast<const float*>(GU), S, m.ffn, L.fatrelu_threshold, n, static_cast<uint2*>(nullptr),
                        static_cast<float2*>(nullptr), static_cast<float*>(nullptr));
            if (st != ASDSL_OK) return st;
            st = mfma ? preq2_fused_batch(L.down_meta, L.down_quant, S, O, m.hidden, m.ffn, m.gs_ffn, n, stream,
                                          true, mimg, w.mimg_bytes)
                      : gemv_exact(L.down_meta, L.down_quant, S, nullptr, O, m.hidden, m.ffn, m.gs_ffn);
        }
        if (st != ASDSL_OK) return st;
        pending = O;
    }
    st = norm_then_gemv(pending, m.rms_out, m.lm_meta, m.lm_quant, logits, m.vocab, m.gs_lm);
    if (st != ASDSL_OK) return st;
    st = launch("verify_argmax_kernel", verify_argmax_kernel, dim3(kArgmaxWgs, n), dim3(256), 0, s,
                static_cast<const float*>(logits), m.vocab, keys);
    if (st != ASDSL_OK) return st;
    return launch("verify_tokens_kernel", verify_tokens_kernel, dim3(1), dim3(kWave), 0, s,
                  static_cast<const unsigned long long*>(keys), next_tokens, n);
}

extern "C" asdsl_status asdsl_kv_zero_from(uint16_t* k_cache, uint16_t* v_cache, int n_kv_heads, int head_dim,
                                           int max_seq, int from_pos, asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(k_cache && v_cache, "kv_zero_from: null pointer");
    ASDSL_CHECK_ARG(head_dim == kHeadDim, "kv_zero_from: head_dim must be 128");
    ASDSL_CHECK_ARG(n_kv_heads > 0 && max_seq > 0, "kv_zero_from: invalid dimensions");
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(k_cache) % 16 == 0 && reinterpret_cast<uintptr_t>(v_cache) % 16 == 0,
                    "kv_zero_from: caches must be 16-byte aligned");
    const int from = from_pos < 0 ? 0 : from_pos;
    if (from >= max_seq) return ASDSL_OK;  // nothing past the cache (zero_kv_from returns too)
    const size_t total = static_cast<size_t>(max_seq - from) * (kHeadDim / 8) * n_kv_heads;
    const unsigned grid = static_cast<unsigned>(total / 256 + 1 < 4096 ? total / 256 + 1 : 4096);
    return launch("kv_zero_kernel", kv_zero_kernel, dim3(grid), dim3(256), 0, as_hip(stream),
                  reinterpret_cast<uint4*>(k_cache), reinterpret_cast<uint4*>(v_cache), n_kv_heads, max_seq, from);
}

extern "C" asdsl_status asdsl_kv_zero_from_q8(int8_t* k_cache, int8_t* v_cache, float* k_scale, float* v_scale,
                                              int n_kv_heads, int head_dim, int max_seq, int from_pos,
                                              asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(k_cache && v_cache && k_scale && v_scale, "kv_zero_from_q8: null pointer");
    ASDSL_CHECK_ARG(head_dim == kHeadDim, "kv_zero_from_q8: head_dim must be 128");
    ASDSL_CHECK_ARG(n_kv_heads > 0 && max_seq > 0, "kv_zero_from_q8: invalid dimensions");
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(k_cache) % 16 == 0 && reinterpret_cast<uintptr_t>(v_cache) % 16 == 0,
                    "kv_zero_from_q8: caches must be 16-byte aligned");
    const int from = from_pos < 0 ? 0 : from_pos;
    if (from >= max_seq) return ASDSL_OK;
    const size_t total = static_cast<size_t>(max_seq - from) * (kHeadDim / 16) * n_kv_heads;
    const unsigned grid = static_cast<unsigned>(total / 256 + 1 < 4096 ? total / 256 + 1 : 4096);
    return launch("kv_zero_q8_kernel", kv_zero_q8_kernel, dim3(grid), dim3(256), 0, as_hip(stream),
                  reinterpret_cast<uint4*>(k_cache), reinterpret_cast<uint4*>(v_cache), k_scale, v_scale, n_kv_heads,
                  max_seq, from);
}

#ifdef ASDSL_WG_TIMELINE
// Timing build only (lib/libasdsl_hip_timeline.so), no reference counterpart:
// the decode step's kernels stamp their workgroup timeline into buf
// (kTimelineSlots * kTimelineWgs * 8 uint64, layout in device_common.hpp);
// null switches the stamps off.
extern "C" asdsl_status asdsl_timeline_set_buffer(void* buf) {
    const hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(asdsl::g_timeline), &buf, sizeof(buf));
    if (e != hipSuccess) {
        asdsl::set_error("timeline: %s", hipGetErrorString(e));
        return ASDSL_ERR_HIP;
    }
    const asdsl_status st = asdsl::timeline_set_preq2(buf);
    return st != ASDSL_OK ? st : asdsl::timeline_set_sparse(buf);
}
#endif
