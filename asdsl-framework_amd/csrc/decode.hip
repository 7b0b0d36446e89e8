// One batch-1 decode step of a Phi-4-shaped model on the GPU: the glue around
// the preq2 GEMVs (embedding, RoPE + KV write + attention over an fp16 KV
// cache, greedy argmax) and the host driver that queues a whole token.
//
// Reference: UnifiedEngine::forward_token (asdsl/kernels/native/unified_engine.cpp:1339-1688)
//   with its helpers load_embed_row_f32 (181-197), rope_apply_inplace (768-801),
//   set_kv_cache (859-920), compute_attention_flash_q8 (922-1027),
//   argmax_f32_avx2 (207-233).  The reference caches K/V as int8 per 64; this
//   step keeps them fp16 (the decode workload's KV format); the current
//   token's K/V are rounded to fp16 before use, as if read back from the cache.
//
// Per layer (6 launches): qkv GEMV with residual add + RMSNorm in its
// prologue, attention partials, attention combine, o_proj GEMV, gate_up GEMV
// with residual add + RMSNorm, down GEMV with SwiGLU in its prologue.  The
// token id and position live in device memory, so a captured graph of one
// step replays token after token with no host work.
#include <hip/hip_fp16.h>

#include "abi_util.hpp"
#include "device_common.hpp"

namespace asdsl {
namespace {

constexpr int kHeadDim = 128;
constexpr int kSplit = 128;        // positions per attention workgroup
constexpr int kAttnThreads = 256;  // 4 waves x 4 positions per step
constexpr int kPartStride = kHeadDim + 2;  // m, l, acc[128]

__device__ __forceinline__ float h2f(uint16_t b) { return __half2float(__ushort_as_half(b)); }
__device__ __forceinline__ uint16_t f2h(float v) { return __half_as_ushort(__float2half_rn(v)); }

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

// Next token = the argmax row; position + 1.
__global__ void finalize_kernel(const unsigned long long* __restrict__ amax, int* __restrict__ token,
                                int* __restrict__ pos) {
    if (threadIdx.x == 0) {
        *token = static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(*amax));
        *pos += 1;
    }
}

// Attention partials of one KV head over positions [s*kSplit, min((s+1)*kSplit, pos+1)).
// G = query heads per KV head.  Lane l of a wave reads dims 8*(l%16).. of
// position 4*step + l/16, so every K/V load instruction moves 1 KiB of
// consecutive positions.  Writes per query head (m, l, acc[128]) with
// acc = sum_p exp(s_p - m) v_p.  The split holding `pos` also applies RoPE to
// the new K, rounds K and V to fp16 and stores them in the cache.
// Each wave keeps its 32 positions' scores in registers and forms its own
// (max, sum, P.V); the four waves are merged in LDS behind one barrier (a
// block-wide softmax through LDS took two more barriers and ~2 us longer).

template <int G>
__global__ __launch_bounds__(kAttnThreads) void attn_partial_kernel(
    const float* __restrict__ qkv, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin, const int* __restrict__ pos_ptr,
    float* __restrict__ part, int n_heads, int n_kv, int max_seq, int rot_half, int nsplit) {
    __shared__ float q_s[G][kHeadDim];
    __shared__ float kv_new[2][kHeadDim];
    __shared__ float wml[kAttnThreads / kWave][G][2];
    __shared__ float wacc[kAttnThreads / kWave][G][kHeadDim];
    const int s = static_cast<int>(blockIdx.x);
    const int kvh = static_cast<int>(blockIdx.y);
    const int pos = *pos_ptr;
    const int p0 = s * kSplit;
    // whole workgroup: this split is past the sequence, or the position is
    // outside the cache (the combine then writes zeros)
    if (p0 > pos || pos < 0 || pos >= max_seq) return;
    const int p1 = min(p0 + kSplit, pos + 1);
    const int tid = static_cast<int>(threadIdx.x);
    const float inv_sqrt_d = 1.0f / sqrtf(static_cast<float>(kHeadDim));
    const int lane = tid & (kWave - 1);
    const int wave = tid >> 6;
    const int pg = lane >> 4;   // position within the wave's four
    const int dc = lane & 15;   // 8-dim chunk
    const size_t head_base = static_cast<size_t>(kvh) * max_seq * kHeadDim;

    // RoPE inputs first (small, from L2), then every K and V row this lane
    // will use (they depend on nothing but pos): loads complete in issue
    // order, so the rotation waits only for its own inputs and the kernel
    // waits on HBM once.  Rows of positions 4*wave + pg + 16*it of the split;
    // `pos` itself comes from LDS.
    const float* cp = rope_cos + static_cast<size_t>(pos) * rot_half;
    const float* sp = rope_sin + static_cast<size_t>(pos) * rot_half;
    constexpr int kRope = ((G + 1) * kHeadDim + kAttnThreads - 1) / kAttnThreads;
    float rx[kRope][4];
#pragma unroll
    for (int r = 0; r < kRope; ++r) {
        const int e = tid + r * kAttnThreads;
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
    constexpr int kIt = kSplit / 16;
    uint4 kraw[kIt], vraw[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
        const int p = p0 + wave * 4 + pg + 16 * it;
        if (p < p1 && p != pos) {
            const size_t at = head_base + static_cast<size_t>(p) * kHeadDim + 8 * dc;
            kraw[it] = *reinterpret_cast<const uint4*>(kc + at);
            vraw[it] = *reinterpret_cast<const uint4*>(vc + at);
        } else {
            kraw[it] = make_uint4(0u, 0u, 0u, 0u);
            vraw[it] = kraw[it];
        }
    }

    // RoPE (half split over the first 2*rot_half dims) on the G query heads
    // and the KV head's new key; the new value as is.
#pragma unroll
    for (int r = 0; r < kRope; ++r) {
        const int e = tid + r * kAttnThreads;
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
            else kv_new[0][d] = h2f(f2h(val));
        }
    }
    if (tid < kHeadDim) kv_new[1][tid] = h2f(f2h(vnew));
    __syncthreads();
    if (pos < p1 && tid < kHeadDim) {
        kc[head_base + static_cast<size_t>(pos) * kHeadDim + tid] = f2h(kv_new[0][tid]);
        vc[head_base + static_cast<size_t>(pos) * kHeadDim + tid] = f2h(kv_new[1][tid]);
    }

    float qr[G][8];
#pragma unroll
    for (int hh = 0; hh < G; ++hh)
#pragma unroll
        for (int e = 0; e < 8; ++e) qr[hh][e] = q_s[hh][8 * dc + e];

    auto row_of = [&](const uint4& raw, int which, int p, float (&r)[8]) {
        if (p == pos) {
#pragma unroll
            for (int e = 0; e < 8; ++e) r[e] = kv_new[which][8 * dc + e];
        } else {
            const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                r[2 * e] = h2f(static_cast<uint16_t>(w[e] & 0xFFFFu));
                r[2 * e + 1] = h2f(static_cast<uint16_t>(w[e] >> 16));
            }
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
    // the wave's max and exp-sum per head (over its iterations, then over the
    // four position groups: lanes 16 apart); a wave with no position keeps
    // m = -inf and l = 0
    float m[G], l[G];
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
        float v = sr[0][hh];
#pragma unroll
        for (int it = 1; it < kIt; ++it) v = fmaxf(v, sr[it][hh]);
        v = fmaxf(v, swz_xor16(v));
        v = fmaxf(v, __shfl_xor(v, 32, kWave));
        m[hh] = v;
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
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
        l[hh] += swz_xor16(l[hh]);
        l[hh] += __shfl_xor(l[hh], 32, kWave);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            acc[hh][e] += swz_xor16(acc[hh][e]);
            acc[hh][e] += __shfl_xor(acc[hh][e], 32, kWave);
        }
    }
    if (pg == 0) {
#pragma unroll
        for (int hh = 0; hh < G; ++hh)
#pragma unroll
            for (int e = 0; e < 8; ++e) wacc[wave][hh][8 * dc + e] = acc[hh][e];
    }
    if (lane == 0) {  // m and l are uniform across the wave
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
            wml[wave][hh][0] = m[hh];
            wml[wave][hh][1] = l[hh];
        }
    }
    __syncthreads();

    // merge the waves: M = max m_w, acc = sum_w exp(m_w - M) acc_w, L likewise
    constexpr int kWaves = kAttnThreads / kWave;
    for (int e = tid; e < G * kHeadDim; e += kAttnThreads) {
        const int hh = e / kHeadDim;
        const int d = e % kHeadDim;
        float M = wml[0][hh][0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) M = fmaxf(M, wml[w][hh][0]);
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float mw = wml[w][hh][0];
            sum = fmaf(mw == -INFINITY ? 0.0f : expf(mw - M), wacc[w][hh][d], sum);
        }
        part[(static_cast<size_t>(kvh * G + hh) * nsplit + s) * kPartStride + 2 + d] = sum;
    }
    if (tid < G) {
        float M = wml[0][tid][0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) M = fmaxf(M, wml[w][tid][0]);
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float mw = wml[w][tid][0];
            L = fmaf(mw == -INFINITY ? 0.0f : expf(mw - M), wml[w][tid][1], L);
        }
        float* pp = part + (static_cast<size_t>(kvh * G + tid) * nsplit + s) * kPartStride;
        pp[0] = M;
        pp[1] = L;
    }
}

// out[h][d] = sum_s e_s acc_s[d] / sum_s e_s l_s, e_s = exp(m_s - max m).
// Up to kCombineGroups groups of 128 threads each fold a contiguous run of
// splits (chunks of kChunk loads issued together, a running (max, sum,
// output) rescaled between chunks); with more than one group the runs are
// merged in LDS in split order.  One group when the splits fit one chunk.
constexpr int kCombineGroups = 4;
constexpr int kCombineThreads = kCombineGroups * kHeadDim;

__global__ __launch_bounds__(kCombineThreads) void attn_combine_kernel(const float* __restrict__ part,
                                                                      const int* __restrict__ pos_ptr,
                                                                      float* __restrict__ out, int nsplit,
                                                                      int max_seq) {
    constexpr int kChunk = 16;
    __shared__ float gml[kCombineGroups][2];
    __shared__ float go[kCombineGroups][kHeadDim];
    const int h = static_cast<int>(blockIdx.x);
    const int d = static_cast<int>(threadIdx.x) % kHeadDim;
    const int g = static_cast<int>(threadIdx.x) / kHeadDim;
    const int pos = *pos_ptr;
    if (pos < 0 || pos >= max_seq) {  // outside the cache: no partials were written
        if (g == 0) out[static_cast<size_t>(h) * kHeadDim + d] = 0.0f;
        return;
    }
    const int ns = pos / kSplit + 1;
    const int ng = min(kCombineGroups, (ns + kChunk - 1) / kChunk);  // groups with splits
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
    if (ng == 1) {  // uniform: group 0 holds every split
        if (g == 0) out[static_cast<size_t>(h) * kHeadDim + d] = o * (1.0f / L);
        return;
    }
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
        out[static_cast<size_t>(h) * kHeadDim + d] = sum * (1.0f / Ls);
    }
}

int attn_splits(int max_seq) { return (max_seq + kSplit - 1) / kSplit; }

asdsl_status launch_attention(const float* qkv, uint16_t* kc, uint16_t* vc, const float* rc, const float* rs,
                              const int* pos, float* att, float* part, int n_heads, int n_kv, int rot_half,
                              int max_seq, hipStream_t s) {
    const int nsplit = attn_splits(max_seq);
    const int G = n_heads / n_kv;
    asdsl_status st;
    const dim3 grid(nsplit, n_kv);
    switch (G) {
        case 1: st = launch("attn_partial_kernel", attn_partial_kernel<1>, grid, dim3(kAttnThreads), 0, s, qkv, kc, vc, rc, rs, pos, part, n_heads, n_kv, max_seq, rot_half, nsplit); break;
        case 2: st = launch("attn_partial_kernel", attn_partial_kernel<2>, grid, dim3(kAttnThreads), 0, s, qkv, kc, vc, rc, rs, pos, part, n_heads, n_kv, max_seq, rot_half, nsplit); break;
        case 3: st = launch("attn_partial_kernel", attn_partial_kernel<3>, grid, dim3(kAttnThreads), 0, s, qkv, kc, vc, rc, rs, pos, part, n_heads, n_kv, max_seq, rot_half, nsplit); break;
        case 4: st = launch("attn_partial_kernel", attn_partial_kernel<4>, grid, dim3(kAttnThreads), 0, s, qkv, kc, vc, rc, rs, pos, part, n_heads, n_kv, max_seq, rot_half, nsplit); break;
        default:
            set_error("attention: n_heads / n_kv_heads must be 1..4");
            return ASDSL_ERR_UNSUPPORTED;
    }
    if (st != ASDSL_OK) return st;
    return launch("attn_combine_kernel", attn_combine_kernel, dim3(n_heads), dim3(kCombineThreads), 0, s,
                  static_cast<const float*>(part), pos, att, nsplit, max_seq);
}

// Work buffer layout of one decode step (offsets in floats, 256-byte aligned).
struct DecodeWork {
    size_t hA, hB, qkv, att, o, gu, down, part, amax, total;
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
    w.part = take(static_cast<size_t>(m.n_heads) * attn_splits(m.max_seq) * kPartStride);
    w.amax = take(2);
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
    return ASDSL_OK;
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

extern "C" size_t asdsl_attention_work_floats(int n_heads, int max_seq) {
    return static_cast<size_t>(n_heads) * attn_splits(max_seq) * kPartStride;
}

extern "C" asdsl_status asdsl_attention_f16kv(const float* qkv, uint16_t* k_cache, uint16_t* v_cache,
                                              const float* rope_cos, const float* rope_sin, const int* pos,
                                              float* att_out, float* work, int n_heads, int n_kv_heads,
                                              int head_dim, int rotary_dim, int max_seq, asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(qkv && k_cache && v_cache && rope_cos && rope_sin && pos && att_out && work,
                    "attention_f16kv: null pointer");
    ASDSL_CHECK_ARG(head_dim == kHeadDim, "attention_f16kv: head_dim must be 128");
    ASDSL_CHECK_ARG(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0 && n_heads / n_kv_heads <= 4,
                    "attention_f16kv: n_heads must be a multiple (1..4x) of n_kv_heads");
    ASDSL_CHECK_ARG(rotary_dim > 0 && rotary_dim % 2 == 0 && rotary_dim <= head_dim,
                    "attention_f16kv: rotary_dim must be even and <= head_dim");
    ASDSL_CHECK_ARG(max_seq > 0, "attention_f16kv: max_seq must be positive");
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(k_cache) % 16 == 0 && reinterpret_cast<uintptr_t>(v_cache) % 16 == 0,
                    "attention_f16kv: caches must be 16-byte aligned");
    return launch_attention(qkv, k_cache, v_cache, rope_cos, rope_sin, pos, att_out, work, n_heads, n_kv_heads,
                            rotary_dim / 2, max_seq, as_hip(stream));
}

extern "C" size_t asdsl_decode_work_bytes(const asdsl_decode_model* model) {
    if (check_model(model) != ASDSL_OK) return 0;
    return decode_work(*model).total * sizeof(float);
}

extern "C" asdsl_status asdsl_decode_token(const asdsl_decode_model* model, int* token, int* pos, float* logits,
                                           void* work, asdsl_stream_t stream) {
    const asdsl_status cs = check_model(model);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(token && pos && logits && work, "decode_token: null pointer");
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
    hipStream_t s = as_hip(stream);
    const int qkv_dim = (m.n_heads + 2 * m.n_kv_heads) * m.head_dim;
    const int q_dim = m.n_heads * m.head_dim;

    asdsl_status st = launch("embed_kernel", embed_kernel, dim3((m.hidden + 1023) / 1024), dim3(256), 0, s,
                             m.embed, static_cast<const int*>(token), hA, m.hidden, m.vocab, amax);
    if (st != ASDSL_OK) return st;
    // The residual stream enters layer l in `cur`; layer l > 0 adds the
    // previous down output in its qkv prologue and writes the sum to `nxt`.
    float* cur = hA;
    float* nxt = hB;
    for (int l = 0; l < m.n_layers; ++l) {
        const asdsl_decode_layer& L = m.layers[l];
        if (l > 0) {
            st = asdsl_gemv_preq2_rmsnorm(L.qkv_meta, L.qkv_quant, cur, down, L.rms_att, nxt, qkv, qkv_dim,
                                          m.hidden, m.gs_attn, m.rms_eps, nullptr, stream);
            std::swap(cur, nxt);
        } else {
            st = asdsl_gemv_preq2_rmsnorm(L.qkv_meta, L.qkv_quant, cur, nullptr, L.rms_att, nullptr, qkv, qkv_dim,
                                          m.hidden, m.gs_attn, m.rms_eps, nullptr, stream);
        }
        if (st != ASDSL_OK) return st;
        st = launch_attention(qkv, L.k_cache, L.v_cache, m.rope_cos, m.rope_sin, pos, att, part, m.n_heads,
                              m.n_kv_heads, m.rotary_dim / 2, m.max_seq, s);
        if (st != ASDSL_OK) return st;
        st = asdsl_gemv_preq2_fused(L.o_meta, L.o_quant, att, o, m.hidden, q_dim, m.gs_attn, stream);
        if (st != ASDSL_OK) return st;
        st = asdsl_gemv_preq2_rmsnorm(L.gu_meta, L.gu_quant, cur, o, L.rms_ffn, nxt, gu, 2 * m.ffn, m.hidden,
                                      m.gs_ffn, m.rms_eps, nullptr, stream);
        if (st != ASDSL_OK) return st;
        std::swap(cur, nxt);
        st = asdsl_gemv_preq2_swiglu(L.down_meta, L.down_quant, gu, down, m.hidden, m.ffn, m.gs_ffn,
                                     L.fatrelu_threshold, stream);
        if (st != ASDSL_OK) return st;
    }
    st = asdsl_gemv_preq2_rmsnorm(m.lm_meta, m.lm_quant, cur, down, m.rms_out, nullptr, logits, m.vocab, m.hidden,
                                  m.gs_lm, m.rms_eps, amax, stream);
    if (st != ASDSL_OK) return st;
    return launch("finalize_kernel", finalize_kernel, dim3(1), dim3(64), 0, s,
                  static_cast<const unsigned long long*>(amax), token, pos);
}
