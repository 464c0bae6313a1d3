// k_router.hip - router logits and top-k gating for gfx950.
//
// Logits: out[t][e] = sum_k W[e][k] * x[t][k], accumulated in binary64 as
// the engine's CPU path does (sf37.c:1970-1976).  Tiled: a workgroup owns
// 32 experts x 32 tokens, stages 64-wide K slices of both operands in LDS
// and each thread accumulates a 2x2 patch in double (shapes the matrix-core
// kernel below does not take); up to 16 tokens a GEMV kernel.
//
// Selection (sf37.c:2144-2157, sf37_cuda.cu:4866-4997): one wave per token.
// p = sigmoid(logit), score = p + bias, k rounds of a wave-wide arg-max under
// (score desc, index asc), weights = p / max(sum p, 1e-20) * scale with the
// sum taken in slot order.
#include "sf37_router.h"
#include "sf37_launch.h"

namespace {

constexpr int RT_E = 32, RT_T = 32, RT_K = 64;

__global__ void __launch_bounds__(256) f32_matmul_kernel(float *__restrict__ out,
                                                         const float *__restrict__ w,
                                                         const float *__restrict__ x,
                                                         uint64_t in_dim, uint64_t out_dim,
                                                         uint64_t n_tok) {
    __shared__ float ws[RT_E][RT_K + 1];
    __shared__ float xs[RT_T][RT_K + 1];
    const uint64_t e0 = (uint64_t)blockIdx.x * RT_E;
    const uint64_t t0 = (uint64_t)blockIdx.y * RT_T;
    const uint32_t tid = threadIdx.x;
    const uint32_t te = (tid & 15u) * 2u, tt = (tid >> 4) * 2u;
    double acc[2][2] = {{0.0, 0.0}, {0.0, 0.0}};
    for (uint64_t k0 = 0; k0 < in_dim; k0 += RT_K) {
        for (uint32_t i = tid; i < RT_E * RT_K; i += 256u) {
            const uint32_t r = i / RT_K, c = i % RT_K;
            const uint64_t e = e0 + r, k = k0 + c;
            ws[r][c] = (e < out_dim && k < in_dim) ? w[e * in_dim + k] : 0.0f;
            const uint64_t t = t0 + r;
            xs[r][c] = (t < n_tok && k < in_dim) ? x[t * in_dim + k] : 0.0f;
        }
        __syncthreads();
#pragma unroll 8
        for (int c = 0; c < RT_K; c++) {
            const double w0 = ws[te][c], w1 = ws[te + 1][c];
            const double x0 = xs[tt][c], x1 = xs[tt + 1][c];
            acc[0][0] = __builtin_fma(w0, x0, acc[0][0]);
            acc[0][1] = __builtin_fma(w0, x1, acc[0][1]);
            acc[1][0] = __builtin_fma(w1, x0, acc[1][0]);
            acc[1][1] = __builtin_fma(w1, x1, acc[1][1]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint64_t e = e0 + te + i, t = t0 + tt + j;
            if (e < out_dim && t < n_tok) out[t * out_dim + e] = (float)acc[i][j];
        }
}

// Prefill logits on the fp64 matrix cores (v_mfma_f64_16x16x4f64): the
// fp32 operands convert exactly to binary64, every product is exact and the
// sums are binary64, so the logits stay within 1 ulp of the CPU's ordered
// sum.  A workgroup owns 32 tokens x RL_E experts (96 when that pads E less
// than 64 does: 288 = 3 x 96) and one of S contiguous K slices, walked in
// 64-wide chunks: x and W rows copied with float4 loads into LDS (rows
// padded by four floats so a step's 16 rows x 4 columns fall in distinct
// banks), the next chunk held in registers while the current one is
// consumed.  Wave w takes tokens 16(w & 1).. and experts RL_E/2 (w >> 1)..,
// RL_E/32 MFMA tiles sharing the token operand; MFMA step s4 takes column
// s4 + l/16 of both operands, so the k index is the same in A and B.
// Token tiles go to the 8 XCDs round-robin (XCD k takes tiles k mod 8), so
// each x row is read by one XCD.  With S > 1 each slice writes its binary64
// partial sums and rl_reduce_kernel adds the slices in slice order (a fixed
// order: the logits do not depend on scheduling); S is chosen so the grid
// holds about three workgroups per CU (at 512 tokens 16 slices: 48 tiles
// alone would leave 208 CUs idle while each walked all of K).
typedef double rt_f64x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t RL_T = 32, RL_K = 64, RL_P = RL_K + 4, RL_MAX_SLICES = 16;

template <uint32_t RL_E>
__global__ void __launch_bounds__(256) f64mm_router_lds_kernel(float *__restrict__ out, double *__restrict__ part,
                                                               const float *__restrict__ w,
                                                               const float *__restrict__ x, uint32_t K, uint32_t E,
                                                               uint32_t T) {
    static_assert(RL_T == 32 && RL_E % 32 == 0 && RL_K % 32 == 0, "copy: 32 rows x 8 float4 lanes per pass");
    constexpr uint32_t RL_WT = RL_E / 32u;     // W rows per copying thread
    __shared__ float xs[2][RL_T * RL_P];
    __shared__ float ws[2][RL_E * RL_P];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t nt = (T + RL_T - 1u) / RL_T, ne = (E + RL_E - 1u) / RL_E;
    const uint32_t xcd = blockIdx.x & 7u, q = blockIdx.x >> 3;
    const uint32_t ct = nt > xcd ? (nt - xcd + 7u) / 8u : 0u;      // token tiles of this XCD
    if (q >= ct * ne) return;
    const uint32_t et = q / ct, tt = xcd + 8u * (q - et * ct);
    const uint32_t t0 = tt * RL_T, e0 = et * RL_E;
    const uint32_t S = gridDim.y, ks = K / S, kb = blockIdx.y * ks;   // this workgroup's K slice
    // copy assignments: x row tid/8 (float4 tid%8); W rows 32m + tid/8
    const uint32_t cr = tid >> 3, cc = (tid & 7u) * 4u;
    const uint32_t xr = t0 + cr < T ? t0 + cr : T - 1u;               // loads stay in bounds
    const float *xp = x + (uint64_t)xr * K + kb + cc;
    const float *wp[RL_WT];
#pragma unroll
    for (uint32_t m = 0; m < RL_WT; m++) {
        const uint32_t wr = e0 + 32u * m + cr < E ? e0 + 32u * m + cr : E - 1u;
        wp[m] = w + (uint64_t)wr * K + kb + cc;
    }
    constexpr uint32_t NC = RL_K / 32u;    // float4 columns per thread and row
    sf37_f32x4 rx[NC], rw[RL_WT][NC];
    auto fetch = [&](uint32_t ko) {
#pragma unroll
        for (uint32_t c = 0; c < NC; c++) {
            rx[c] = *(const sf37_f32x4 *)(xp + ko + 32u * c);
#pragma unroll
            for (uint32_t m = 0; m < RL_WT; m++) rw[m][c] = *(const sf37_f32x4 *)(wp[m] + ko + 32u * c);
        }
    };
    auto stage = [&](uint32_t buf) {
#pragma unroll
        for (uint32_t c = 0; c < NC; c++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                xs[buf][cr * RL_P + 32u * c + cc + j] = rx[c][j];
#pragma unroll
                for (uint32_t m = 0; m < RL_WT; m++) ws[buf][(32u * m + cr) * RL_P + 32u * c + cc + j] = rw[m][c][j];
            }
    };
    fetch(0);
    stage(0);
    __syncthreads();
    const uint32_t i = lane & 15u, g = lane >> 4;
    constexpr uint32_t NT = RL_E / 32u;    // 16-expert MFMA tiles per wave
    const uint32_t ta = (wave & 1u) * 16u + i, eb = (wave >> 1) * (RL_E / 2u) + i;
    rt_f64x4 acc[NT];
#pragma unroll
    for (uint32_t h = 0; h < NT; h++) acc[h] = rt_f64x4{0.0, 0.0, 0.0, 0.0};
    const uint32_t nk = ks / RL_K;
    for (uint32_t kc = 0; kc < nk; kc++) {
        const uint32_t buf = kc & 1u;
        if (kc + 1u < nk) fetch((kc + 1u) * RL_K);
        const float *xa = &xs[buf][ta * RL_P + g];
        const float *wa = &ws[buf][eb * RL_P + g];
#pragma unroll
        for (uint32_t s4 = 0; s4 < RL_K; s4 += 4u) {
            const double a = (double)xa[s4];
#pragma unroll
            for (uint32_t h = 0; h < NT; h++)
                acc[h] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, (double)wa[16u * h * RL_P + s4], acc[h], 0, 0, 0);
        }
        if (kc + 1u < nk) {
            stage(buf ^ 1u);
        }
        __syncthreads();
    }
    // D: lane l holds rows l/16 + 4r (tokens), column l%16 (expert)
    double *ps = part + (uint64_t)blockIdx.y * T * E;
#pragma unroll
    for (uint32_t h = 0; h < NT; h++) {
        const uint32_t e = e0 + (wave >> 1) * (RL_E / 2u) + 16u * h + i;
#pragma unroll
        for (uint32_t r = 0; r < 4; r++) {
            const uint32_t t = t0 + (wave & 1u) * 16u + g + 4u * r;
            if (t < T && e < E) {
                if (S == 1u) out[(uint64_t)t * E + e] = (float)acc[h][r];
                else ps[(uint64_t)t * E + e] = acc[h][r];
            }
        }
    }
}

// out[j] = the S slices' binary64 partial sums added in slice order, rounded once.
__global__ void __launch_bounds__(256) rl_reduce_kernel(float *__restrict__ out, const double *__restrict__ part,
                                                        uint32_t S, uint64_t n) {
    const uint64_t j = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (j >= n) return;
    double v = part[j];
    for (uint32_t s = 1; s < S; s++) v += part[(uint64_t)s * n + j];
    out[j] = (float)v;
}

// Decode GEMV (n_tok small): one workgroup per expert row and 8 tokens.
// For in_dim a multiple of 256 the row is split into contiguous per-thread
// slices (sf37_router.h, the order the fused decode path uses); otherwise
// thread i takes k = i, i + 256, ...  Binary64 partial sums per wave are
// combined as (w0 + w1) + (w2 + w3).
__global__ void __launch_bounds__(256) f32_matvec_kernel(float *__restrict__ out,
                                                         const float *__restrict__ w,
                                                         const float *__restrict__ x,
                                                         uint64_t in_dim, uint64_t out_dim,
                                                         uint32_t n_tok) {
    constexpr int MAXT = 8;
    __shared__ double part[MAXT][4];
    const uint64_t e = blockIdx.x;
    const uint32_t t0 = blockIdx.y * MAXT;
    const uint32_t nt = n_tok - t0 < (uint32_t)MAXT ? n_tok - t0 : (uint32_t)MAXT;
    const float *wr = w + e * in_dim;
    if (in_dim % 256u == 0 && in_dim <= 0xffffffffu) {
        sf37_router_rows(wr, x + (uint64_t)t0 * in_dim, (uint32_t)in_dim, nt, part);
    } else {
        double acc[MAXT];
#pragma unroll
        for (int t = 0; t < MAXT; t++) acc[t] = 0.0;
        for (uint64_t k = threadIdx.x; k < in_dim; k += 256u) {
            const double wv = wr[k];
#pragma unroll
            for (int t = 0; t < MAXT; t++)
                if ((uint32_t)t < nt) acc[t] = __builtin_fma(wv, (double)x[(uint64_t)(t0 + t) * in_dim + k], acc[t]);
        }
#pragma unroll
        for (int t = 0; t < MAXT; t++) {
            double v = acc[t];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
            if ((threadIdx.x & 63u) == 0) part[t][threadIdx.x >> 6] = v;
        }
    }
    __syncthreads();
    if (threadIdx.x < nt) {
        const uint32_t t = threadIdx.x;
        out[(uint64_t)(t0 + t) * out_dim + e] = sf37_router_combine(part[t]);
    }
}

__global__ void __launch_bounds__(256) router_select_kernel(int32_t *__restrict__ selected,
                                                            float *__restrict__ weights,
                                                            float *__restrict__ probs,
                                                            const float *__restrict__ logits,
                                                            const double *__restrict__ part, uint32_t S,
                                                            const float *__restrict__ bias,
                                                            uint32_t n_experts, uint32_t topk,
                                                            float scale, uint32_t n_tok) {
    __shared__ uint64_t tab[32];
    sf37_stage_exp_tab(tab);
    __syncthreads();
    const uint32_t t = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (t >= n_tok) return;
    int32_t *so[1] = {selected + (uint64_t)t * topk};
    float *wo[1] = {weights + (uint64_t)t * topk};
    float *po[1] = {probs ? probs + (uint64_t)t * n_experts : nullptr};
    if (part) {
        // logits left as S binary64 slices by the split router GEMM: added in
        // slice order and rounded once, as rl_reduce_kernel does
        const uint64_t n = (uint64_t)n_tok * n_experts;
        const double *pt = part + (uint64_t)t * n_experts;
        sf37_wave_topk<1>(
            [pt, n, S](uint32_t, uint32_t e) {
                double v = pt[e];
                for (uint32_t k = 1; k < S; k++) v += pt[(uint64_t)k * n + e];
                return (float)v;
            },
            bias, n_experts, topk, scale, tab, so, wo, po);
    } else {
        const float *lg = logits + (uint64_t)t * n_experts;
        sf37_wave_topk<1>([lg](uint32_t, uint32_t e) { return lg[e]; }, bias, n_experts, topk, scale, tab, so, wo, po);
    }
}

uint32_t router_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    return (uint32_t)cus;
}

// Matrix-core plan for n_tok > 16: expert tile (96 or 64, the one that pads
// E less) and the number of K slices (a power of two up to 16 that divides K
// into 64-wide chunks, the smallest giving about three workgroups per CU).
// Returns 0 where the GEMV or the generic kernel runs instead.
int rl_plan(uint64_t in_dim, uint64_t out_dim, uint64_t n_tok, uint32_t *te, uint32_t *S) {
    if (n_tok <= 16 || in_dim % 128u != 0 || in_dim > 0xffffffffu || out_dim > 0xffffffffu || n_tok > 0xffffffffu)
        return 0;
    const uint64_t pad96 = (out_dim + 95) / 96 * 96 - out_dim, pad64 = (out_dim + 63) / 64 * 64 - out_dim;
    *te = pad96 <= pad64 ? 96u : 64u;
    const uint64_t tiles = (n_tok + RL_T - 1) / RL_T * ((out_dim + *te - 1) / *te), want = 3u * router_cus();
    uint32_t s = 1;
    while (s < RL_MAX_SLICES && tiles * s < want && in_dim % (2u * s * RL_K) == 0) s *= 2u;
    *S = s;
    return 1;
}

}  // namespace

extern "C" uint64_t sf37k_f32_matmul_part_bytes(uint64_t in_dim, uint64_t out_dim, uint64_t n_tok) {
    uint32_t te, S;
    return rl_plan(in_dim, out_dim, n_tok, &te, &S) && S > 1u ? (uint64_t)S * n_tok * out_dim * 8u : 0u;
}

extern "C" int sf37k_f32_matmul(float *out, const float *w, const float *x, uint64_t in_dim,
                                uint64_t out_dim, uint64_t n_tok, double *part, uint64_t part_bytes,
                                uint32_t *slices_left, sf37_stream_t s) {
    if (slices_left) *slices_left = 1;
    if (out_dim == 0 || n_tok == 0) return 0;
    uint32_t te, S;
    if (n_tok <= 16) {
        hipLaunchKernelGGL(f32_matvec_kernel, dim3((unsigned)out_dim, (unsigned)((n_tok + 7) / 8)),
                           dim3(256), 0, (hipStream_t)s, out, w, x, in_dim, out_dim, (uint32_t)n_tok);
    } else if (rl_plan(in_dim, out_dim, n_tok, &te, &S)) {
        if (S > 1u && (!part || part_bytes < (uint64_t)S * n_tok * out_dim * 8u)) S = 1;   // no workspace: one slice
        const uint64_t nt = (n_tok + RL_T - 1) / RL_T, ne = (out_dim + te - 1) / te;
        const dim3 grid((unsigned)(8u * ((nt + 7) / 8) * ne), S);
        if (te == 96u)
            hipLaunchKernelGGL(f64mm_router_lds_kernel<96>, grid, dim3(256), 0, (hipStream_t)s, out, part, w, x,
                               (uint32_t)in_dim, (uint32_t)out_dim, (uint32_t)n_tok);
        else
            hipLaunchKernelGGL(f64mm_router_lds_kernel<64>, grid, dim3(256), 0, (hipStream_t)s, out, part, w, x,
                               (uint32_t)in_dim, (uint32_t)out_dim, (uint32_t)n_tok);
        if (S > 1u && slices_left) {
            *slices_left = S;   // the caller's top-8 launch adds the slices
        } else if (S > 1u) {
            const uint64_t n = n_tok * out_dim;
            hipLaunchKernelGGL(rl_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)s, out,
                               (const double *)part, S, n);
        }
    } else {
        hipLaunchKernelGGL(f32_matmul_kernel,
                           dim3((unsigned)((out_dim + RT_E - 1) / RT_E), (unsigned)((n_tok + RT_T - 1) / RT_T)),
                           dim3(256), 0, (hipStream_t)s, out, w, x, in_dim, out_dim, n_tok);
    }
    return (int)hipGetLastError();
}

extern "C" int sf37k_router_select(int32_t *selected, float *weights, float *probs,
                                   const float *logits, const float *bias, uint32_t n_experts,
                                   uint32_t topk, float scale, uint32_t n_tok, sf37_stream_t s) {
    return sf37k_router_select_part(selected, weights, probs, logits, NULL, 1, bias, n_experts, topk, scale, n_tok, s);
}

extern "C" int sf37k_router_select_part(int32_t *selected, float *weights, float *probs, const float *logits,
                                        const double *part, uint32_t slices, const float *bias, uint32_t n_experts,
                                        uint32_t topk, float scale, uint32_t n_tok, sf37_stream_t s) {
    if (n_tok == 0) return 0;
    hipLaunchKernelGGL(router_select_kernel, dim3((n_tok + 3) / 4), dim3(256), 0, (hipStream_t)s, selected,
                       weights, probs, logits, slices > 1u ? part : (const double *)NULL, slices, bias, n_experts,
                       topk, scale, n_tok);
    return (int)hipGetLastError();
}
