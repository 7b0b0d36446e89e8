// preq2 Q4 GEMV for gfx950 (4-row band layout + sidecar fp16 scale/zero).
//
// Reference: gemv_preq2_fused_avx2 / gemv_preq2_avx2
//   (asdsl/kernels/native/gemv_preq2_avx2.cpp:196-337), layout
//   asdsl/quantization/repack_preq2.py:22-62.
//
// Mapping.  A band (4 output rows) is K/8 contiguous 16-byte units.  A
// workgroup of WAVES waves works on WAVES/KS bands at a time; the KS waves of
// one band split its units into contiguous slices of NU*64, lane l of a slice
// owning units slice+l, slice+l+64, ... so each load instruction moves 1 KiB of
// contiguous HBM.  A lane's units always sit at the same K positions, whatever
// band it works on, so the activation units it needs are read from LDS into
// registers once, after the workgroup has quantized x, and reused for every
// band.  64 is a multiple of 4*(GS/32), so a lane always sees the same row slot
// (and, for g128, the same 32-element quarter of its group); row sums fall out
// of a butterfly over the other lane bits (DPP + swizzle + one bpermute), and
// the KS slices are added in a fixed order through LDS: results are
// deterministic.
//
// Launch shape (measured on MI355X, rotated weights): fat workgroups (8 waves,
// 16 when K > 4096 or when 16-band tiles give about one per compute unit)
// amortize the per-workgroup activation quantization, which for K=8192 reads
// more bytes than the workgroup's own weights when workgroups are small; KS
// grows only while fewer than CUs/2 workgroups would be launched.  o_proj
// 3072x3072 3.0 us (KS=2), gate_up 16384x3072 6.75 us (KS=1, 16 waves),
// down 3072x8192 5.1 us (KS=4, 12 waves).
//
// The activation loads are issued before the weight loads (vmcnt retires in
// order) and quantized while the weights are in flight; the next tile's loads
// are issued right after the current tile's dots.
//
// Math per unit (32 elements), fp32 after an exact int32 dot:
//   acc += D*(s*xs) - (z*s)*(X*xs)
// the reference's per-group term (gemv_preq2_avx2.cpp:168-191) with
// D = sum q*xq, X = sum xq.  y is overwritten.
#include "abi_util.hpp"
#include "device_common.hpp"

namespace asdsl {

namespace {

constexpr int kThreads = 256;  // helper kernels
ASDSL_TIMELINE_BUFFER

// Decode-step work fused into the GEMV's activation prologue / epilogue.
//   kNorm:   h = x (+ delta); workgroup 0 writes h to h_out (the new residual
//            stream); the GEMV input is rmsnorm(h) = (h * inv_rms) * nw with
//            inv_rms = 1/sqrt(sum(h^2)/K + eps)
//            (residual_add_rmsnorm_f32 / rmsnorm_f32, unified_engine.cpp:499-524,651-688),
//            computed as inv_rms * GEMV(h * nw) (the factor moved past the
//            quantizer, see the prologue).
//   kSwiglu: the GEMV input is silu(x) * up, zeroed where |value| < thr when
//            thr > 0 (swiglu_inplace with fast_exp_avx2, unified_engine.cpp:803-857).
//   kCombine: the GEMV input is the attention output, merged here from the
//            split partials when the position has at most pa.fold splits
//            (attn_combine_kernel then skipped that position), with that
//            kernel's single-group arithmetic operation for operation, so the
//            input is bit for bit the one it would have written; otherwise x,
//            which it did write.
//   ARGMAX:  the largest output and its row (first on ties, as argmax_f32_avx2,
//            unified_engine.cpp:207-233) are folded into *amax with a 64-bit
//            atomicMax: key = order-preserving float bits << 32 | ~row, so the
//            result does not depend on workgroup order.  *amax must be zero
//            before the launch.
//   kNormEmbed: kNorm whose h is the fp16 embedding row of *pa.token (a
//            token outside [0, vocab) reads row 0), converted to fp32;
//            workgroup 0 stores h to h_out and clears *pa.amax (the step's
//            argmax key) (load_embed_row_f32, unified_engine.cpp:181-197).
enum class Pro { kPlain, kNorm, kSwiglu, kCombine, kNormEmbed };

constexpr int kMaxFold = 8;  // kCombine: most splits merged in the prologue

struct ProArgs {
    const float* delta = nullptr;
    const float* nw = nullptr;
    float* h_out = nullptr;
    const float* up = nullptr;
    unsigned long long* amax = nullptr;
    float eps = 0.0f;
    float thr = 0.0f;
    // kNorm / kNormEmbed: quantize (h * inv_rms) * nw, the reference's
    // order (0), or h * nw with the outputs scaled by inv_rms (1: the
    // factored form, preq2_norm_factored())
    int norm_factored = 0;
    // kCombine: partials [head][split][m, l, acc[head_dim]] (part_stride
    // floats each, nsplit rows per head), the position and the split policy:
    // nt = pos / tile + 1 tiles, tps = ceil(nt / max_splits) tiles per split,
    // ceil(nt / tps) splits
    const float* part = nullptr;
    const int* pos = nullptr;
    int nsplit = 0, tile = 0, max_splits = 0, part_stride = 0, head_dim = 0, max_seq = 0;
    int pos_limit = 0x7FFFFFFF;  // positions at or past it had no partials written
    // SWIGLU_EPI: the output rows are [gate F | up F] with F = 4 * fbands;
    // y receives swiglu(gate, up) (F values, pa.thr applies)
    int fbands = 0;
    // kNormEmbed: fp16 embedding table [vocab][K] and the token id (device)
    const uint16_t* embed = nullptr;
    const int* token = nullptr;
    int vocab = 0;
};

// Units of a lane's first tile requested before the activation is staged,
// by split code: 0 all of them, 1 a third, 2 a half, 3 two thirds (rounded
// up); the rest are requested once the activation is staged.
template <int NU, int SPLIT>
constexpr int pre_units() {
    return SPLIT == 0 ? NU : SPLIT == 1 ? (NU + 2) / 3 : SPLIT == 2 ? (NU + 1) / 2 : (2 * NU + 2) / 3;
}

// Block sum in fixed order, in two halves around a barrier the caller
// already has: each wave's butterfly sum to s_red[wave], then, after the
// barrier, the waves' sums in wave order.
__device__ __forceinline__ void wave_sum_to_lds(float v, float* s_red) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
    if ((threadIdx.x & (kWave - 1)) == 0) s_red[threadIdx.x >> 6] = v;
}

template <int WAVES>
__device__ __forceinline__ float sum_waves(const float* s_red) {
    float t = s_red[0];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) t += s_red[w];
    return t;
}

template <int GS, int NU, int WAVES, int NCH, bool Q8, bool EXACT, bool XREG, Pro PRO = Pro::kPlain,
          bool ARGMAX = false, bool SWIGLU_EPI = false, int SPLIT = 0>
__global__ __launch_bounds__(WAVES * kWave) void preq2_gemv_kernel(const uint32_t* __restrict__ meta,
                                                                  const uint4* __restrict__ quant,
                                                                  const float* __restrict__ x,
                                                                  const int8_t* __restrict__ xq8,
                                                                  const float* __restrict__ xsc,
                                                                  float* __restrict__ y, int M, int K, int lks,
                                                                  ProArgs pa) {
    extern __shared__ __align__(16) uint32_t lds[];
    __shared__ float s_part[2][WAVES][4];
    constexpr int kTl = PRO == Pro::kCombine                 ? 0
                        : SWIGLU_EPI                         ? 1
                        : (PRO == Pro::kNorm && !ARGMAX)     ? 2
                        : (PRO == Pro::kPlain && !Q8)        ? (WAVES > 8 ? 3 : 7)
                                                             : -1;
    const int tl_wg = static_cast<int>(blockIdx.x);
    ASDSL_TIMELINE_STAMP(kTl, tl_wg, 0);
    constexpr int UPS = GS / 32;       // units per (row, group)
    constexpr int UPG4 = 4 * UPS;      // units per (band, group)
    constexpr int SB = UPS == 1 ? 0 : 2;
    const int G = K / GS;
    const XImage im = x_image(lds, K, GS);

    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int KS = 1 << lks;
    const int ks = wave & (KS - 1);
    const int bl = wave >> lks;
    const int bpt = WAVES >> lks;      // bands per tile
    const int nbands = (M + 3) >> 2;
    // SWIGLU_EPI (KS = 1): tile t pairs gate bands t*h .. t*h+h-1 (waves
    // 0..h-1) with the up bands fbands + t*h .. (waves h..2h-1), h = bpt/2,
    // so every gate row meets its up row in the workgroup
    const int hpt = bpt >> 1;
    const int ntiles = SWIGLU_EPI ? (pa.fbands + hpt - 1) / hpt : (nbands + bpt - 1) / bpt;
    auto band_of = [&](int t) {
        if constexpr (SWIGLU_EPI) return bl < hpt ? t * hpt + bl : pa.fbands + t * hpt + (bl - hpt);
        else return t * bpt + bl;
    };
    const int upb = K >> 3;            // units per band
    const int c0 = ks * (NU * kWave) + lane;
    const int part = lane % UPS;
    const int slot = (lane / UPS) & 3;
    const bool writer = lane < UPG4 && part == 0;

    // This lane's units.  EXACT (KS*NU*64 == K/8): every unit is in the band
    // and sits at a constant offset from the first.  Otherwise indices are
    // clamped in bounds and units past the band are masked.
    int cu[NU];
    bool valid[NU];
#pragma unroll
    for (int j = 0; j < NU; ++j) {
        valid[j] = EXACT || c0 + j * kWave < upb;
        cu[j] = EXACT ? c0 + j * kWave : min(c0 + j * kWave, upb - 1);
    }

    uint4 w[NU];
    uint32_t mt[NU];
    // Loads are unconditional at in-bounds indices; values of rows >= M
    // (tail band) are never stored.
    // units lo .. hi-1 of a tile (uniform bounds)
    auto load_tile = [&](int tile, int lo, int hi) {
        const int band = min(band_of(tile), nbands - 1);
        const uint4* qb = quant + static_cast<size_t>(band) * upb;
        const int row = min(band * 4 + slot, M - 1);
        const uint32_t* mrow = meta + static_cast<size_t>(row) * G;
        if (EXACT) {
            const uint4* qp = qb + c0;
            const uint32_t* mp = mrow + c0 / UPG4;
#pragma unroll
            for (int j = 0; j < NU; ++j)
                if (j >= lo && j < hi) w[j] = load_stream16(qp + j * kWave);
#pragma unroll
            for (int j = 0; j < NU; ++j)
                if (j >= lo && j < hi) mt[j] = mp[j * (kWave / UPG4)];
        } else {
#pragma unroll
            for (int j = 0; j < NU; ++j)
                if (j >= lo && j < hi) w[j] = load_stream16(qb + cu[j]);
#pragma unroll
            for (int j = 0; j < NU; ++j)
                if (j >= lo && j < hi) mt[j] = mrow[cu[j] / UPG4];
        }
    };

    int tile = static_cast<int>(blockIdx.x);
    const int tile_step = static_cast<int>(gridDim.x);
    ActStage<GS, WAVES * kWave, NCH, Q8> act;
    const int nchunk = K >> 3;
    const int tid = static_cast<int>(threadIdx.x);
    static_assert(PRO != Pro::kCombine || (NCH == 1 && !Q8), "kCombine: one fp32 chunk per thread");
    constexpr int NF = PRO == Pro::kCombine ? kMaxFold : 1;
    float2 fml[NF];    // kCombine: (m, l) of each split
    float fav[NF][8];  // kCombine: this thread's 8 accumulator values of each split
    int fns = 0;       // kCombine: splits merged here (0: x holds the merged output)
    if constexpr (PRO == Pro::kCombine) {
        const int p = *pa.pos;
        if (p >= 0 && p < pa.max_seq && p < pa.pos_limit) {
            const int nt = p / pa.tile + 1;
            const int tps = (nt + pa.max_splits - 1) / pa.max_splits;
            fns = (nt + tps - 1) / tps;  // <= max_splits <= kMaxFold
        }
        if (fns > 0) {
            const int e0 = min(tid, nchunk - 1) * 8;  // this thread's 8 outputs: head h, dims d0..d0+7
            const int h = e0 / pa.head_dim;
            const int d0 = e0 - h * pa.head_dim;
            const float* ph = pa.part + static_cast<size_t>(h) * pa.nsplit * pa.part_stride;
#pragma unroll
            for (int sp = 0; sp < NF; ++sp) {
                if (sp < fns) {
                    const float* pp = ph + static_cast<size_t>(sp) * pa.part_stride;
                    fml[sp] = *reinterpret_cast<const float2*>(pp);
                    const float2* a2 = reinterpret_cast<const float2*>(pp + 2 + d0);
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const float2 t = a2[k];
                        fav[sp][2 * k] = t.x;
                        fav[sp][2 * k + 1] = t.y;
                    }
                }
            }
        }
    }
    constexpr bool kNormed = PRO == Pro::kNorm || PRO == Pro::kNormEmbed;
    if constexpr (PRO == Pro::kNormEmbed) {  // the embedding row, fp16 -> fp32
        const int t0 = *pa.token;
        const int t = t0 >= 0 && t0 < pa.vocab ? t0 : 0;
        const uint4* row = reinterpret_cast<const uint4*>(pa.embed + static_cast<size_t>(t) * K);
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const uint4 u = row[min(i * WAVES * kWave + tid, nchunk - 1)];
            const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                act.v[i][2 * e] = half_bits_to_float(w4[e]);
                act.v[i][2 * e + 1] = half_bits_to_float(w4[e] >> 16);
            }
        }
        if (blockIdx.x == 0 && tid == 0 && pa.amax) *pa.amax = 0ull;
    } else if (fns == 0) {
        act.load(x, xq8, xsc, K);  // activation loads first: they retire first
    }
    constexpr int NX = PRO == Pro::kPlain || PRO == Pro::kCombine ? 1 : NCH;
    float ex[NX][8], ew[NX][8];  // kNorm: delta, norm weight; kSwiglu: up
    if constexpr (kNormed || PRO == Pro::kSwiglu) {
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int c = min(i * WAVES * kWave + tid, nchunk - 1);
            const float* src0 = kNormed ? pa.delta : pa.up;
#pragma unroll
            for (int e = 0; e < 8; ++e) ex[i][e] = 0.0f;
            if (PRO != Pro::kNormEmbed && src0) {
                const float4 a = reinterpret_cast<const float4*>(src0)[2 * c];
                const float4 b = reinterpret_cast<const float4*>(src0)[2 * c + 1];
                ex[i][0] = a.x; ex[i][1] = a.y; ex[i][2] = a.z; ex[i][3] = a.w;
                ex[i][4] = b.x; ex[i][5] = b.y; ex[i][6] = b.z; ex[i][7] = b.w;
            }
            if constexpr (kNormed) {
                const float4 a = reinterpret_cast<const float4*>(pa.nw)[2 * c];
                const float4 b = reinterpret_cast<const float4*>(pa.nw)[2 * c + 1];
                ew[i][0] = a.x; ew[i][1] = a.y; ew[i][2] = a.z; ew[i][3] = a.w;
                ew[i][4] = b.x; ew[i][5] = b.y; ew[i][6] = b.z; ew[i][7] = b.w;
            }
        }
    }
    // 16-wave workgroups: every wave's activation requests go
    // out before any wave's weight requests.  A CU returns vector-memory data
    // in request order, so activation loads queued behind other waves' weight
    // misses wait for HBM, and the staging barrier below waits for the
    // slowest wave (down 3072x8192: 5.55 -> 5.24 us; at 8 waves it measured
    // ~1 % slower, so it is not done there).  The barrier waits on nothing
    // outstanding.
    if constexpr (WAVES > 8) __syncthreads();
    // grid <= ntiles, so this tile exists.  SPLIT: only the first units go
    // out now, the rest once the activation is staged (below), so that the
    // activation is not queued behind the launch's whole weight stream.
    constexpr int kPre = pre_units<NU, SPLIT>();
    load_tile(tile, 0, kPre);
    // kNorm: the GEMV input is rmsnorm(h) = (h * inv_rms) * nw, quantized
    // per group as the reference's rmsnorm + quantize_activation form it;
    // the block sum of squares (fixed order) is reduced behind an extra
    // barrier before the quantization.  The factored form
    // (pa.norm_factored) skips that barrier: 1/rms is one positive factor of
    // the whole input, so the codes of h * nw are those of the normed input
    // up to fp32 rounding (a quotient within rounding of a .5 boundary can
    // take the other code) and the GEMV of h * nw scaled by inv_rms is the
    // GEMV of the normed input; it quantizes h * nw at once and scales its
    // reduced outputs by inv_rms.
    __shared__ float s_red[kNormed ? WAVES : 1];
    if constexpr (kNormed) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int c = i * WAVES * kWave + tid;
#pragma unroll
            for (int e = 0; e < 8; ++e) act.v[i][e] += ex[i][e];
            if (c < nchunk) {
#pragma unroll
                for (int e = 0; e < 8; ++e) ss = fmaf(act.v[i][e], act.v[i][e], ss);
                if (pa.h_out && blockIdx.x == 0) {
                    reinterpret_cast<float4*>(pa.h_out)[2 * c] =
                        make_float4(act.v[i][0], act.v[i][1], act.v[i][2], act.v[i][3]);
                    reinterpret_cast<float4*>(pa.h_out)[2 * c + 1] =
                        make_float4(act.v[i][4], act.v[i][5], act.v[i][6], act.v[i][7]);
                }
            }
        }
        wave_sum_to_lds(ss, s_red);
        if (pa.norm_factored) {  // uniform per launch
#pragma unroll
            for (int i = 0; i < NCH; ++i)
#pragma unroll
                for (int e = 0; e < 8; ++e) act.v[i][e] *= ew[i][e];
        } else {
            __syncthreads();
            const float inv = 1.0f / sqrtf(sum_waves<WAVES>(s_red) / static_cast<float>(K) + pa.eps);
#pragma unroll
            for (int i = 0; i < NCH; ++i)
#pragma unroll
                for (int e = 0; e < 8; ++e) act.v[i][e] = (act.v[i][e] * inv) * ew[i][e];
        }
    } else if constexpr (PRO == Pro::kSwiglu) {
#pragma unroll
        for (int i = 0; i < NCH; ++i)
#pragma unroll
            for (int e = 0; e < 8; ++e) act.v[i][e] = swiglu_ref(act.v[i][e], ex[i][e], pa.thr);
    } else if constexpr (PRO == Pro::kCombine) {
        if (fns > 0) {  // one group over splits 0..fns-1: running max, then e-weighted sums
            float cm = -INFINITY;
#pragma unroll
            for (int sp = 0; sp < NF; ++sp)
                if (sp < fns) cm = fmaxf(cm, fml[sp].x);
            float L = 0.0f;
            float o[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) o[k] = 0.0f;
#pragma unroll
            for (int sp = 0; sp < NF; ++sp) {
                if (sp < fns) {
                    const float e = expf(fml[sp].x - cm);
                    L = fmaf(e, fml[sp].y, L);
#pragma unroll
                    for (int k = 0; k < 8; ++k) o[k] = fmaf(e, fav[sp][k], o[k]);
                }
            }
            const float inv = 1.0f / L;
#pragma unroll
            for (int k = 0; k < 8; ++k) act.v[0][k] = o[k] * inv;
        }
    }
    act.process(K, im);        // quantize while the weights are in flight
    if constexpr (kPre < NU) {
        __builtin_amdgcn_sched_barrier(0);  // keep these requests behind the staging
        load_tile(tile, kPre, NU);
    }
    ASDSL_TIMELINE_STAMP(kTl, tl_wg, 1);
    __syncthreads();
    ASDSL_TIMELINE_STAMP(kTl, tl_wg, 2);
    float inv_rms = 1.0f;  // the factored form's output scale (1 otherwise: an exact multiply)
    if constexpr (kNormed) {
        if (pa.norm_factored) inv_rms = 1.0f / sqrtf(sum_waves<WAVES>(s_red) / static_cast<float>(K) + pa.eps);
    }

    // XREG: this lane's activation units are copied from LDS into registers
    // once and reused for every tile; otherwise they are read per tile.
    uint32_t xr[XREG ? NU : 1][8];
    float xs[XREG ? NU : 1], xu[XREG ? NU : 1];
    auto read_x = [&](int j, uint32_t (&dst)[8], float& sc, float& us) {
        const int g = cu[j] / UPG4;
        const int u = g * UPS + part;
        const uint4 a = reinterpret_cast<const uint4*>(im.xq + u * 8)[0];
        const uint4 b = reinterpret_cast<const uint4*>(im.xq + u * 8)[1];
        dst[0] = a.x; dst[1] = a.y; dst[2] = a.z; dst[3] = a.w;
        dst[4] = b.x; dst[5] = b.y; dst[6] = b.z; dst[7] = b.w;
        sc = im.scale[g];
        us = im.usum[u];
    };
    if (XREG) {
#pragma unroll
        for (int j = 0; j < NU; ++j) read_x(j, xr[XREG ? j : 0], xs[XREG ? j : 0], xu[XREG ? j : 0]);
    }

    int parity = 0;
    unsigned long long best = 0;  // ARGMAX: this thread's largest key
    for (; tile < ntiles; tile += tile_step) {  // uniform per workgroup
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            if (valid[j]) {
                uint32_t xt[8];
                float sc, us;
                if (!XREG) read_x(j, xt, sc, us);
                const int jj = XREG ? j : 0;
                const int d = unit_dot(w[j], XREG ? xr[jj] : xt);
                const float s = half_bits_to_float(mt[j]);
                const float z = half_bits_to_float(mt[j] >> 16);
                acc = fmaf(static_cast<float>(d), s * (XREG ? xs[jj] : sc), acc);
                acc = fmaf(-(z * s), XREG ? xu[jj] : us, acc);
            }
        }
        if (tile == static_cast<int>(blockIdx.x)) ASDSL_TIMELINE_STAMP(kTl, tl_wg, 3);
        const int band = band_of(tile);
        acc = slot_sum<SB>(acc);
        if constexpr (kNormed) acc *= inv_rms;
        // next tile's loads after the reduction: issuing them before it keeps
        // ~20 more VGPRs live (measured), costing a workgroup per CU at NU=6
        if (tile + tile_step < ntiles) load_tile(tile + tile_step, 0, NU);
        const int row = band * 4 + slot;
        if constexpr (SWIGLU_EPI) {
            // the up waves hand their rows to the gate waves through LDS (two
            // buffers by tile parity: one barrier per tile suffices)
            __shared__ float s_up[2][WAVES / 2][4];
            if (bl >= hpt && writer) s_up[parity][bl - hpt][slot] = acc;
            __syncthreads();
            if (bl < hpt && writer && band < pa.fbands)
                y[row] = swiglu_ref(acc, s_up[parity][bl][slot], pa.thr);
            parity ^= 1;
        } else if (lks == 0) {
            if (writer && band < nbands && row < M) {
                y[row] = acc;
                if constexpr (ARGMAX) best = max(best, argmax_key(acc, row));
            }
        } else {
            if (writer) s_part[parity][wave][slot] = acc;
            __syncthreads();
            if (ks == 0 && writer && band < nbands && row < M) {
                float sum = s_part[parity][wave][slot];
                for (int k = 1; k < KS; ++k) sum += s_part[parity][wave + k][slot];
                y[row] = sum;
                if constexpr (ARGMAX) best = max(best, argmax_key(sum, row));
            }
            parity ^= 1;
        }
    }
    ASDSL_TIMELINE_STAMP(kTl, tl_wg, 4);
    if constexpr (ARGMAX) {
        // max is order-free: any reduction order gives the same key.  One
        // atomic per workgroup (one per wave serialized on the single address:
        // measured 2x the whole lm_head).
        __shared__ unsigned long long s_best[WAVES];
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            const uint32_t lo = __shfl_xor(static_cast<uint32_t>(best), o, kWave);
            const uint32_t hi = __shfl_xor(static_cast<uint32_t>(best >> 32), o, kWave);
            best = max(best, (static_cast<unsigned long long>(hi) << 32) | lo);
        }
        if (lane == 0) s_best[wave] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long b = s_best[0];
#pragma unroll
            for (int w = 1; w < WAVES; ++w) b = max(b, s_best[w]);
            if (b != 0) atomicMax(pa.amax, b);
        }
    }
}

// w[r*K + k] = (q - z) * s, one thread per unit.
template <int GS>
__global__ __launch_bounds__(kThreads) void preq2_dequant_kernel(const uint32_t* __restrict__ meta,
                                                                const uint4* __restrict__ quant,
                                                                float* __restrict__ out, int M, int K) {
    constexpr int UPS = GS / 32;
    const int U = K >> 5;
    const int G = K / GS;
    const long long total = static_cast<long long>(M) * U;
    for (long long t = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; t < total;
         t += static_cast<long long>(gridDim.x) * kThreads) {
        const int r = static_cast<int>(t / U);
        const int u = static_cast<int>(t % U);
        const int g = u / UPS;
        const int part = u % UPS;
        const int band = r >> 2;
        const int slot = r & 3;
        const size_t unit = static_cast<size_t>(band) * (U * 4) + static_cast<size_t>(g) * (4 * UPS) + slot * UPS + part;
        const uint4 wq = quant[unit];
        const uint32_t m = meta[static_cast<size_t>(r) * G + g];
        const float s = half_bits_to_float(m);
        const float z = half_bits_to_float(m >> 16);
        const uint32_t wv[4] = {wq.x, wq.y, wq.z, wq.w};
        float* o = out + static_cast<size_t>(r) * K + static_cast<size_t>(u) * 32;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float4 a, b;
            a.x = (static_cast<float>(wv[i] & 0xF) - z) * s;
            a.y = (static_cast<float>((wv[i] >> 4) & 0xF) - z) * s;
            a.z = (static_cast<float>((wv[i] >> 8) & 0xF) - z) * s;
            a.w = (static_cast<float>((wv[i] >> 12) & 0xF) - z) * s;
            b.x = (static_cast<float>((wv[i] >> 16) & 0xF) - z) * s;
            b.y = (static_cast<float>((wv[i] >> 20) & 0xF) - z) * s;
            b.z = (static_cast<float>((wv[i] >> 24) & 0xF) - z) * s;
            b.w = (static_cast<float>((wv[i] >> 28) & 0xF) - z) * s;
            reinterpret_cast<float4*>(o)[2 * i] = a;
            reinterpret_cast<float4*>(o)[2 * i + 1] = b;
        }
    }
}

// Standalone activation quantizer (natural int8 order out); each workgroup
// quantizes a run of kThreads chunks.
template <int GS>
__global__ __launch_bounds__(kThreads) void quantize_activation_kernel(const float* __restrict__ x,
                                                                      int8_t* __restrict__ xq,
                                                                      float* __restrict__ xs, int K) {
    __shared__ __align__(16) uint32_t s_split[2 * kThreads];
    __shared__ float s_scale[kThreads];
    __shared__ float s_sum[kThreads];
    const XImage im{s_split, s_scale, s_sum};
    const int nchunk = K >> 3;
    for (int base = static_cast<int>(blockIdx.x) * kThreads; base < nchunk;
         base += static_cast<int>(gridDim.x) * kThreads) {  // uniform per workgroup
        const int c = base + static_cast<int>(threadIdx.x);
        const bool active = c < nchunk;
        float v[8];
        if (active) {
            const float4 a = reinterpret_cast<const float4*>(x)[2 * c];
            const float4 b = reinterpret_cast<const float4*>(x)[2 * c + 1];
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = 0.0f;
        }
        // chunk index relative to `base` keeps the LDS image small; groups
        // never straddle `base` because kThreads*8 is a multiple of GS.
        quantize_chunk<GS>(v, c - base, active, im, xq + static_cast<size_t>(base) * 8, xs + base * 8 / GS);
    }
}

int check_preq2_args(const void* meta, const void* quant, const void* x, const void* y, int M, int K, int gs,
                     const char* fn) {
    if (!meta || !quant || !x || !y) {
        set_error("%s: null pointer", fn);
        return 1;
    }
    if (gs != 32 && gs != 128) {
        set_error("%s: group_size must be 32 (preq2) or 128 (preq2-g128)", fn);
        return 1;
    }
    if (M <= 0 || K <= 0) {
        set_error("%s: invalid dimensions", fn);
        return 1;
    }
    if (K % gs != 0) {
        set_error("%s: in_features must be divisible by group_size", fn);
        return 1;
    }
    if (K / 32 > 640) {
        set_error("%s: n_groups exceeds buffer", fn);
        return 1;
    }
    return 0;
}

// Launch plan.  waves: 8 per workgroup, 16 when K > 4096 (the activation is
// then 32+ KB of fp32 per workgroup), 12 where that fills the compute units
// better (below).  KS: the smallest power of two that
// leaves each lane at most 6 units (loads) per band; then doubled, while it
// splits the band evenly, as long as fewer than CUs/2 workgroups would run.
// ASDSL_HIP_KSPLIT forces KS (a power of two <= 8; raised where the forced
// value would leave more than 6 units per lane); it changes the fp32
// summation order, not the formula.
struct Plan {
    int lks, nu, waves, grid;
    bool exact;
    int split;  // pre_units split code of the first tile's weight requests
};

Plan plan_preq2(int M, int K, int cus, int gs) {
    const int upb = K / 8;
    const int nbands = (M + 3) / 4;
    Plan p{0, 0, K > 4096 ? 16 : 8, 0, false, 0};
    // K <= 4096 where 16-band tiles number between 3/4 of the compute units
    // and all of them (gate_up 16384 rows: 256): 16 waves, one tile per
    // workgroup and one workgroup per compute unit, whose waves all request
    // the activation before any weight (see the kernel), instead of two
    // 8-wave workgroups whose second one's activation waits behind the first
    // one's weights (gate_up 16384x3072: 6.95 -> 6.75 and 6.86 -> 6.75 us on
    // two boxes).  Where a workgroup walks several tiles the staging is
    // amortized and 16 waves measured slower (lm_head 200064x3072 g128: 50.8
    // -> 52.7 us).  ASDSL_HIP_PREQ2_WAVES (read per call) forces 8 or 16.
    const int tiles16 = (nbands + 15) / 16;
    if (K <= 4096 && 4 * tiles16 >= 3 * cus && tiles16 <= cus) p.waves = 16;
    const int forced_waves = env_knob("ASDSL_HIP_PREQ2_WAVES");
    if (forced_waves == 8 || forced_waves == 16) p.waves = forced_waves;
    auto nu_of = [&](int lks) { return (upb + (kWave << lks) - 1) / (kWave << lks); };
    auto tiles_of = [&](int lks) {
        const int bpt = p.waves >> lks;
        return (nbands + bpt - 1) / bpt;
    };
    const int forced = env_knob("ASDSL_HIP_KSPLIT");  // read per call (a test sets it in-process)
    if (forced == 1 || forced == 2 || forced == 4 || forced == 8) {
        p.lks = forced == 1 ? 0 : forced == 2 ? 1 : forced == 4 ? 2 : 3;
        // never more than 6 units per lane (the kernel's largest NU); K/32 <=
        // 640 keeps KS = 8 within it
        while (p.lks < 3 && nu_of(p.lks) > 6) ++p.lks;
    } else {
        while (p.lks < 3 && nu_of(p.lks) > 6) ++p.lks;
        while (p.lks < 3 && tiles_of(p.lks) < cus / 2 && upb % (kWave << (p.lks + 1)) == 0) ++p.lks;
    }
    // K > 4096 at KS = 4: 12 waves (3 bands a tile) instead of 16 when that
    // fills every compute unit with one workgroup where 16 would leave a
    // quarter idle (down 3072x8192: 256 instead of 192 workgroups, 5.28 ->
    // 5.11 us)
    const int nb3 = nbands / 3;
    if (forced == 0 && p.waves == 16 && p.lks == 2 && nbands % 3 == 0 && nbands / 4 < cus && nb3 <= cus)
        p.waves = 12;
    p.nu = nu_of(p.lks);
    p.exact = p.nu * (kWave << p.lks) == upb;
    const int cap = cus * (32 / p.waves);  // at most 32 waves per compute unit
    const int tiles = tiles_of(p.lks);
    p.grid = tiles < cap ? tiles : cap;
    // The activation waits in the memory queues behind the weight requests
    // issued before it, so its arrival grows with the bytes a launch
    // requests up front (1.3 us at 5.9 MB, 3-6 us at 31.5 MB).  From 8 MB of
    // weights the first tile's requests are split around the staging: half
    // of them first below 16 MB, a third from 16 MB (measured: qkv 9.9 MB
    // 4.25 -> 3.87 us, down 15.8 MB 5.08 -> 4.76, gate_up 31.5 MB 7.03 ->
    // 6.81; o_proj 5.9 MB is slower split).  ASDSL_HIP_PRE_SPLIT (read per
    // call) sets the code instead: 1 a third, 2 a half, 4 none.
    const double bytes = static_cast<double>(M) * K * (0.5 + 4.0 / gs);
    p.split = bytes < 8e6 ? 0 : bytes < 16e6 ? 2 : 1;
    const int forced_split = env_knob("ASDSL_HIP_PRE_SPLIT");
    if (forced_split == 1 || forced_split == 2) p.split = forced_split;
    if (forced_split == 4) p.split = 0;
    return p;
}

template <int GS, int WAVES, int NCH, bool Q8, bool EXACT, Pro PRO = Pro::kPlain, bool ARGMAX = false,
          bool SWI = false>
asdsl_status launch_exact(const Plan& p, const uint32_t* m, const uint4* q, const float* x, const int8_t* xq8,
                          const float* xsc, float* y, int M, int K, hipStream_t stream, const ProArgs& pa = ProArgs{}) {
    const size_t lds = x_image_bytes(K, GS);
    const dim3 block(WAVES * kWave);
    constexpr bool XREG = true;
#define ASDSL_PREQ2_NU(N, SPLIT)                                                                                 \
    case N:                                                                                                       \
        return launch("preq2_gemv_kernel",                                                                        \
                      preq2_gemv_kernel<GS, N, WAVES, NCH, Q8, EXACT, XREG, PRO, ARGMAX, SWI, SPLIT>, dim3(p.grid), \
                      block, lds, stream, m, q, x, xq8, xsc, y, M, K, p.lks, pa);
#define ASDSL_PREQ2_NUS(SPLIT)      \
    switch (p.nu) {                 \
        ASDSL_PREQ2_NU(1, SPLIT)    \
        ASDSL_PREQ2_NU(2, SPLIT)    \
        ASDSL_PREQ2_NU(3, SPLIT)    \
        ASDSL_PREQ2_NU(4, SPLIT)    \
        ASDSL_PREQ2_NU(5, SPLIT)    \
        default: ASDSL_PREQ2_NU(6, SPLIT) \
    }
    if constexpr (EXACT && !Q8) {  // the split forms are built for the fp32-input shapes K tiles exactly
        switch (p.split) {
            case 1: ASDSL_PREQ2_NUS(1)
            case 2: ASDSL_PREQ2_NUS(2)
            default: break;
        }
    }
    ASDSL_PREQ2_NUS(0)
#undef ASDSL_PREQ2_NUS
#undef ASDSL_PREQ2_NU
}

template <int GS, int WAVES, int NCH, bool Q8, Pro PRO = Pro::kPlain, bool ARGMAX = false>
asdsl_status launch_waves(const Plan& p, const uint32_t* m, const uint4* q, const float* x, const int8_t* xq8,
                          const float* xsc, float* y, int M, int K, hipStream_t stream, const ProArgs& pa = ProArgs{}) {
    if (p.exact) return launch_exact<GS, WAVES, NCH, Q8, true, PRO, ARGMAX>(p, m, q, x, xq8, xsc, y, M, K, stream, pa);
    return launch_exact<GS, WAVES, NCH, Q8, false, PRO, ARGMAX>(p, m, q, x, xq8, xsc, y, M, K, stream, pa);
}

// gate_up with the residual add + RMSNorm prologue and the SwiGLU epilogue:
// rows [gate F | up F] -> y[F] = swiglu(gate, up).  Needs one wave per band
// (KS = 1) and F/4 divisible by half the bands of a tile; returns
// ASDSL_ERR_UNSUPPORTED (nothing launched) otherwise.
template <int GS>
asdsl_status launch_gateup_swiglu(const uint8_t* meta, const uint8_t* quant, const float* x, float* y, int F, int K,
                                  ProArgs pa, hipStream_t stream, int cus) {
    Plan p = plan_preq2(2 * F, K, cus, GS);
    // 8 waves with two tiles per workgroup (below) unless forced: 16 waves
    // with one tile each measured 957 against 939 us per 32-layer step at
    // ctx 128 (the same bits: a row's sum does not depend on the waves)
    if (p.waves == 16 && K <= 4096 && env_knob("ASDSL_HIP_PREQ2_WAVES") != 16) p.waves = 8;
    const int hpt = (p.waves >> p.lks) / 2;
    if (p.lks != 0 || hpt < 1 || F % 4 != 0 || (F / 4) % hpt != 0) return ASDSL_ERR_UNSUPPORTED;
    pa.fbands = F / 4;
    const int tiles = (F / 4) / hpt;
    const int cap = cus * (32 / p.waves);
    // Two tiles per workgroup (the second requested after the first's
    // reduction): half as many workgroups stage the activation (each reads h,
    // delta and the norm weights, 36 KiB at hidden 3072), measured 11-13 us
    // per 32-layer step faster at ctx 128 and 1024 than one tile per
    // workgroup; requesting both tiles up front measured slower.
    // ASDSL_HIP_GATEUP_TILES sets the tiles per workgroup.
    // (16-wave workgroups hold twice the bands: one tile each keeps one
    // workgroup per compute unit.)
    static const int tpw_knob = env_knob("ASDSL_HIP_GATEUP_TILES");
    const int tpw = tpw_knob > 0 ? tpw_knob : p.waves == 16 ? 1 : 2;
    const int want = (tiles + tpw - 1) / tpw;
    p.grid = want < cap ? want : cap;
    const auto* m = reinterpret_cast<const uint32_t*>(meta);
    const auto* q = reinterpret_cast<const uint4*>(quant);
    if (p.waves == 8) {
        return p.exact ? launch_exact<GS, 8, 1, false, true, Pro::kNorm, false, true>(p, m, q, x, nullptr, nullptr, y,
                                                                                       2 * F, K, stream, pa)
                       : launch_exact<GS, 8, 1, false, false, Pro::kNorm, false, true>(p, m, q, x, nullptr, nullptr,
                                                                                        y, 2 * F, K, stream, pa);
    }
    return p.exact ? launch_exact<GS, 16, 1, false, true, Pro::kNorm, false, true>(p, m, q, x, nullptr, nullptr, y,
                                                                                    2 * F, K, stream, pa)
                   : launch_exact<GS, 16, 1, false, false, Pro::kNorm, false, true>(p, m, q, x, nullptr, nullptr, y,
                                                                                     2 * F, K, stream, pa);
}

// Decode-step variants (fp32 activation, one chunk per thread: K <= 8192).
template <int GS, Pro PRO, bool ARGMAX>
asdsl_status launch_preq2_fused(const uint8_t* meta, const uint8_t* quant, const float* x, float* y, int M, int K,
                                const ProArgs& pa, hipStream_t stream, int cus) {
    const Plan p = plan_preq2(M, K, cus, GS);
    const auto* m = reinterpret_cast<const uint32_t*>(meta);
    const auto* q = reinterpret_cast<const uint4*>(quant);
    if (p.waves == 8) return launch_waves<GS, 8, 1, false, PRO, ARGMAX>(p, m, q, x, nullptr, nullptr, y, M, K, stream, pa);
    if constexpr (PRO != Pro::kCombine) {  // kCombine stages one chunk per thread
        if (p.waves == 12)
            return launch_waves<GS, 12, 2, false, PRO, ARGMAX>(p, m, q, x, nullptr, nullptr, y, M, K, stream, pa);
    }
    return launch_waves<GS, 16, 1, false, PRO, ARGMAX>(p, m, q, x, nullptr, nullptr, y, M, K, stream, pa);
}

template <int GS, bool Q8>
asdsl_status launch_preq2(const uint8_t* meta, const uint8_t* quant, const float* x, const int8_t* xq8,
                          const float* xsc, float* y, int M, int K, hipStream_t stream, int cus) {
    const Plan p = plan_preq2(M, K, cus, GS);
    const auto* m = reinterpret_cast<const uint32_t*>(meta);
    const auto* q = reinterpret_cast<const uint4*>(quant);
    // one 8-element activation chunk per thread and pass: NCH = ceil(K / (8 * threads))
    if (p.waves == 8) return launch_waves<GS, 8, 1, Q8>(p, m, q, x, xq8, xsc, y, M, K, stream);
    if (p.waves == 12) return launch_waves<GS, 12, 2, Q8>(p, m, q, x, xq8, xsc, y, M, K, stream);
    if (K <= 8192) return launch_waves<GS, 16, 1, Q8>(p, m, q, x, xq8, xsc, y, M, K, stream);
    if (K <= 16384) return launch_waves<GS, 16, 2, Q8>(p, m, q, x, xq8, xsc, y, M, K, stream);
    return launch_waves<GS, 16, 3, Q8>(p, m, q, x, xq8, xsc, y, M, K, stream);
}

}  // namespace

bool preq2_norm_factored() { return env_knob("ASDSL_HIP_NORM_FACTORED") > 0; }

void preq2_plan_shape(int M, int K, int cus, int* lks, int* nu, int* waves, bool* exact) {
    const Plan p = plan_preq2(M, K, cus, 32);  // the split code does not change the shape
    *lks = p.lks;
    *nu = p.nu;
    *waves = p.waves;
    *exact = p.exact;
}

#ifdef ASDSL_WG_TIMELINE
asdsl_status timeline_set_preq2(void* buf) {
    const hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(g_timeline), &buf, sizeof(buf));
    if (e != hipSuccess) {
        set_error("timeline: %s", hipGetErrorString(e));
        return ASDSL_ERR_HIP;
    }
    return ASDSL_OK;
}
#endif

}  // namespace asdsl

using namespace asdsl;

extern "C" asdsl_status asdsl_gemv_preq2_fused(const uint8_t* meta, const uint8_t* quant, const float* x, float* y,
                                               int out_features, int in_features, int group_size,
                                               asdsl_stream_t stream) {
    if (check_preq2_args(meta, quant, x, y, out_features, in_features, group_size, "gemv_preq2_fused"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CU_COUNT(cus);
    if (group_size == 32)
        return launch_preq2<32, false>(meta, quant, x, nullptr, nullptr, y, out_features, in_features, as_hip(stream), cus);
    return launch_preq2<128, false>(meta, quant, x, nullptr, nullptr, y, out_features, in_features, as_hip(stream), cus);
}

extern "C" asdsl_status asdsl_gemv_preq2_rmsnorm(const uint8_t* meta, const uint8_t* quant, const float* h_in,
                                                 const float* delta, const float* norm_w, float* h_out, float* y,
                                                 int out_features, int in_features, int group_size, float eps,
                                                 unsigned long long* argmax_key, asdsl_stream_t stream) {
    if (check_preq2_args(meta, quant, h_in, y, out_features, in_features, group_size, "gemv_preq2_rmsnorm"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(norm_w != nullptr, "gemv_preq2_rmsnorm: null norm weight");
    ASDSL_CHECK_ARG(in_features <= 8192, "gemv_preq2_rmsnorm: in_features must be <= 8192");
    ASDSL_CHECK_ARG(h_out == nullptr || (h_out != h_in && h_out != delta),
                    "gemv_preq2_rmsnorm: h_out must not alias h_in or delta (other workgroups still read them)");
    ASDSL_CU_COUNT(cus);
    ProArgs pa;
    pa.delta = delta;
    pa.nw = norm_w;
    pa.norm_factored = preq2_norm_factored() ? 1 : 0;
    pa.h_out = h_out;
    pa.eps = eps;
    pa.amax = argmax_key;
    hipStream_t s = as_hip(stream);
    const int M = out_features, K = in_features;
    if (group_size == 32)
        return argmax_key ? launch_preq2_fused<32, Pro::kNorm, true>(meta, quant, h_in, y, M, K, pa, s, cus)
                          : launch_preq2_fused<32, Pro::kNorm, false>(meta, quant, h_in, y, M, K, pa, s, cus);
    return argmax_key ? launch_preq2_fused<128, Pro::kNorm, true>(meta, quant, h_in, y, M, K, pa, s, cus)
                      : launch_preq2_fused<128, Pro::kNorm, false>(meta, quant, h_in, y, M, K, pa, s, cus);
}

asdsl_status asdsl::preq2_embed_rmsnorm(const uint8_t* meta, const uint8_t* quant, const uint16_t* embed,
                                        const int* token, int vocab, const float* norm_w, float* h_out, float* y,
                                        int out_features, int in_features, int group_size, float eps,
                                        unsigned long long* clear_key, asdsl_stream_t stream) {
    if (check_preq2_args(meta, quant, embed, y, out_features, in_features, group_size, "gemv_preq2_embed_rmsnorm"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(norm_w && token && h_out && vocab > 0, "gemv_preq2_embed_rmsnorm: null pointer");
    ASDSL_CHECK_ARG(in_features <= 8192 && in_features % 8 == 0 && reinterpret_cast<uintptr_t>(embed) % 16 == 0,
                    "gemv_preq2_embed_rmsnorm: in_features must be <= 8192 and the table 16-byte aligned");
    ASDSL_CU_COUNT(cus);
    ProArgs pa;
    pa.nw = norm_w;
    pa.norm_factored = preq2_norm_factored() ? 1 : 0;
    pa.h_out = h_out;
    pa.eps = eps;
    pa.amax = clear_key;
    pa.embed = embed;
    pa.token = token;
    pa.vocab = vocab;
    hipStream_t s = as_hip(stream);
    const float* none = nullptr;
    if (group_size == 32)
        return launch_preq2_fused<32, Pro::kNormEmbed, false>(meta, quant, none, y, out_features, in_features, pa, s, cus);
    return launch_preq2_fused<128, Pro::kNormEmbed, false>(meta, quant, none, y, out_features, in_features, pa, s, cus);
}

asdsl_status asdsl::preq2_fused_combine(const uint8_t* meta, const uint8_t* quant, const float* att, float* y,
                                        int out_features, int in_features, int group_size, const float* part,
                                        const int* pos, int nsplit, int tile, int max_splits, int part_stride,
                                        int head_dim, int max_seq, int pos_limit, asdsl_stream_t stream) {
    if (check_preq2_args(meta, quant, att, y, out_features, in_features, group_size, "gemv_preq2_combine"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(in_features <= 8192, "gemv_preq2_combine: in_features must be <= 8192");
    ASDSL_CHECK_ARG(part && pos && max_splits >= 1 && max_splits <= kMaxFold && max_splits <= nsplit && tile > 0 &&
                        head_dim % 8 == 0 && in_features % head_dim == 0 && part_stride % 2 == 0 &&
                        part_stride >= head_dim + 2 && reinterpret_cast<uintptr_t>(part) % 8 == 0,
                    "gemv_preq2_combine: invalid partial layout");
    ASDSL_CU_COUNT(cus);
    ProArgs pa;
    pa.part = part;
    pa.pos = pos;
    pa.nsplit = nsplit;
    pa.tile = tile;
    pa.max_splits = max_splits;
    pa.part_stride = part_stride;
    pa.head_dim = head_dim;
    pa.max_seq = max_seq;
    pa.pos_limit = pos_limit;
    hipStream_t s = as_hip(stream);
    if (group_size == 32)
        return launch_preq2_fused<32, Pro::kCombine, false>(meta, quant, att, y, out_features, in_features, pa, s, cus);
    return launch_preq2_fused<128, Pro::kCombine, false>(meta, quant, att, y, out_features, in_features, pa, s, cus);
}

extern "C" asdsl_status asdsl_gemv_preq2_rmsnorm_swiglu(const uint8_t* meta, const uint8_t* quant, const float* h_in,
                                                        const float* delta, const float* norm_w, float* h_out,
                                                        float* s_out, int ffn, int in_features, int group_size,
                                                        float eps, float threshold, asdsl_stream_t stream) {
    if (check_preq2_args(meta, quant, h_in, s_out, 2 * ffn, in_features, group_size, "gemv_preq2_rmsnorm_swiglu"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(norm_w != nullptr, "gemv_preq2_rmsnorm_swiglu: null norm weight");
    ASDSL_CHECK_ARG(in_features <= 8192, "gemv_preq2_rmsnorm_swiglu: in_features must be <= 8192");
    ASDSL_CHECK_ARG(ffn > 0 && ffn % 16 == 0, "gemv_preq2_rmsnorm_swiglu: ffn must be a positive multiple of 16");
    ASDSL_CHECK_ARG(h_out == nullptr || (h_out != h_in && h_out != delta),
                    "gemv_preq2_rmsnorm_swiglu: h_out must not alias h_in or delta");
    ASDSL_CU_COUNT(cus);
    ProArgs pa;
    pa.delta = delta;
    pa.nw = norm_w;
    pa.norm_factored = preq2_norm_factored() ? 1 : 0;
    pa.h_out = h_out;
    pa.eps = eps;
    pa.thr = threshold;
    hipStream_t s = as_hip(stream);
    const asdsl_status st = group_size == 32
                                ? launch_gateup_swiglu<32>(meta, quant, h_in, s_out, ffn, in_features, pa, s, cus)
                                : launch_gateup_swiglu<128>(meta, quant, h_in, s_out, ffn, in_features, pa, s, cus);
    if (st == ASDSL_ERR_UNSUPPORTED) set_error("gemv_preq2_rmsnorm_swiglu: no paired gate/up tiling for this shape");
    return st;
}

extern "C" asdsl_status asdsl_gemv_preq2_swiglu(const uint8_t* meta, const uint8_t* quant, const float* gate_up,
                                                float* y, int out_features, int in_features, int group_size,
                                                float threshold, asdsl_stream_t stream) {
    if (check_preq2_args(meta, quant, gate_up, y, out_features, in_features, group_size, "gemv_preq2_swiglu"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(in_features <= 8192, "gemv_preq2_swiglu: in_features must be <= 8192");
    ASDSL_CU_COUNT(cus);
    ProArgs pa;
    pa.up = gate_up + in_features;
    pa.thr = threshold;
    hipStream_t s = as_hip(stream);
    if (group_size == 32)
        return launch_preq2_fused<32, Pro::kSwiglu, false>(meta, quant, gate_up, y, out_features, in_features, pa, s, cus);
    return launch_preq2_fused<128, Pro::kSwiglu, false>(meta, quant, gate_up, y, out_features, in_features, pa, s, cus);
}

extern "C" asdsl_status asdsl_gemv_preq2(const uint8_t* meta, const uint8_t* quant, const int8_t* x_q8,
                                         const float* x_scales, float* y, int out_features, int in_features,
                                         int group_size, asdsl_stream_t stream) {
    if (check_preq2_args(meta, quant, x_q8, y, out_features, in_features, group_size, "gemv_preq2"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(x_scales != nullptr, "gemv_preq2: null pointer");
    ASDSL_CU_COUNT(cus);
    if (group_size == 32)
        return launch_preq2<32, true>(meta, quant, nullptr, x_q8, x_scales, y, out_features, in_features, as_hip(stream), cus);
    return launch_preq2<128, true>(meta, quant, nullptr, x_q8, x_scales, y, out_features, in_features, as_hip(stream), cus);
}

extern "C" asdsl_status asdsl_dequant_preq2(const uint8_t* meta, const uint8_t* quant, float* w, int out_features,
                                            int in_features, int group_size, asdsl_stream_t stream) {
    if (check_preq2_args(meta, quant, w, w, out_features, in_features, group_size, "dequant_preq2"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CU_COUNT(cus);
    const long long units = static_cast<long long>(out_features) * (in_features / 32);
    const int grid = stream_grid(units, kThreads, 16, cus);
    const auto* m = reinterpret_cast<const uint32_t*>(meta);
    const auto* q = reinterpret_cast<const uint4*>(quant);
    return launch("preq2_dequant_kernel", group_size == 32 ? preq2_dequant_kernel<32> : preq2_dequant_kernel<128>,
                  dim3(grid), dim3(kThreads), 0, as_hip(stream), m, q, w, out_features, in_features);
}

extern "C" asdsl_status asdsl_quantize_activation(const float* x, int8_t* x_q8, float* x_scales, int in_features,
                                                  int group_size, asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(x && x_q8 && x_scales, "quantize_activation: null pointer");
    ASDSL_CHECK_ARG(group_size == 32 || group_size == 64 || group_size == 128,
                    "quantize_activation: group_size must be 32, 64 or 128");
    ASDSL_CHECK_ARG(in_features > 0 && in_features % group_size == 0,
                    "quantize_activation: in_features must be a positive multiple of group_size");
    ASDSL_CU_COUNT(cus);
    const int nchunk = in_features / 8;
    const int grid = stream_grid(nchunk, kThreads, 1, cus);
    auto* kernel = group_size == 32   ? quantize_activation_kernel<32>
                   : group_size == 64 ? quantize_activation_kernel<64>
                                      : quantize_activation_kernel<128>;
    return launch("quantize_activation_kernel", kernel, dim3(grid), dim3(kThreads), 0, as_hip(stream), x, x_q8,
                  x_scales, in_features);
}
