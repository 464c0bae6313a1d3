// k_prefill.hip - routed experts for many tokens per expert (prefill) on
// the gfx950 matrix cores.
//
// Same results as the grouped dot-product kernels of k_moe.hip, bit for bit:
// the integer group sums I_g = sum (q - zp) * qs are formed by
// v_mfma_f32_32x32x16_f16 on operands that hold small integers exactly, and
// the float epilogue is the canonical chain of the Q8_K path
//   blk = fma(s3,I3, fma(s2,I2, fma(s1,I1, fma(s0,I0,0))));  acc = fma(d_b, blk, acc)
// (sf37_cuda.cu:4226-4274 sums the same integers; this build fixes the order).
//
// Exactness.  A weight code pair is turned into one dword of two fp16 values
// with a mask and an add: the codes sit in the mantissas under a fixed
// exponent, so each half equals  B + (q - zp)  for a power-of-two bias B that
// depends only on the element's position (fp16 exponent 25 - p for a code at
// mantissa bit p).  Activation codes qs are int8, exact in fp16.  The MFMA
// accumulator starts at  C = -sum_e B_e * qs_e  (a per-token, per-group
// integer the activation kernel precomputes), so it ends at exactly I_g; all
// partial sums are integers below 2^24 in magnitude, hence exact in fp32 in
// any summation order.
//
// Layouts.  Activations are re-quantised to Q8_K (sf37_cuda.cu:4168-4205,
// bit-exact) and written as fp16 codes in the MFMA lane order of the weight
// format, plus a table per (row, 256-block): C of the four 64-groups and d.
// A workgroup owns (tile of <= 128 pairs of one expert, row tile); it stages
// the tile's activation blocks in LDS by direct global->LDS loads (two
// buffers, one block ahead) and each wave streams its own weight rows into
// registers one block ahead, dequantises them in registers and runs the
// MFMAs: 4 token blocks x one 32-column weight block per wave.
#include <type_traits>

#include "sf37_blocks.h"
#include "sf37_launch.h"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr uint32_t PF_T = 64;           // pairs per tile
constexpr uint32_t PF_TB = PF_T / 32u;  // 32-pair MFMA blocks per tile
// Waves per workgroup (32 weight columns each) and activation buffers:
// gate/up one 8-wave workgroup per CU (two waves per SIMD), activations
// three buffers deep; down two 4-wave workgroups per CU (their barriers do
// not stall each other's SIMDs), two buffers.  Measured: 4-wave down
// workgroups 649 against 696 us at 4096 tokens; 4-wave gate/up 1307
// against 1263 us.
template <bool Q3> struct pf_cfg {
    static constexpr uint32_t NW = Q3 ? 8u : 4u;
    static constexpr uint32_t NBUF = Q3 ? 3u : 2u;
    static constexpr uint32_t ROWS = (Q3 ? 16u : 32u) * NW;   // F rows (gate/up) or output rows per workgroup
};
constexpr uint32_t PF_GU_R = pf_cfg<true>::ROWS;    // 128
constexpr uint32_t PF_DN_R = pf_cfg<false>::ROWS;   // 128
constexpr uint32_t PF_CD_ROWS = 8;                  // table rows of LDS per buffer (5 used)
constexpr uint32_t PF_TAB = 8;          // floats per (row, block) table entry: C0..C3, d
// pf_expert table loads (dword): one row of PF_T floats per load, at row
// index wave (8 waves, wave <= 7) or max(wave, 4) (4 waves).
static_assert(PF_T * 4u == 256u, "a table load (64 dwords) writes exactly one row");
static_assert(pf_cfg<true>::NW <= PF_CD_ROWS && pf_cfg<false>::NW <= PF_CD_ROWS && 4u < PF_CD_ROWS,
              "pf_expert table rows stay in their buffer");
// LDS layout of one activation block: 4 groups of 32 tile slots; in a group
// slot t (0..31) starts at PF_RS * (t % 16) + 512 * (t / 16), so one 64-lane
// load fills slots t and t + 16 (512 contiguous bytes each) and 16
// consecutive slots sit 16 bytes apart modulo 256 (no bank conflicts).
constexpr uint32_t PF_RS = 2u * SF37_QK * 2u + 16u;  // 1040
constexpr uint32_t PF_GRP = 16u * PF_RS;             // bytes of 32 slots
constexpr uint32_t PF_ACT_BUF = PF_TB * PF_GRP;      // bytes of one LDS activation block

// Extents of the LDS direct loads.  A global_load_lds writes its 64 lanes'
// bytes at M0 + 16 * lane (dwordx4) or M0 + 4 * lane (dword) whatever the
// source address, so every M0 a kernel forms must leave a whole 64-lane span
// inside the buffer it targets.
constexpr uint32_t DMA16_SPAN = 64u * 16u;
constexpr uint32_t DMA4_SPAN = 64u * 4u;
// pf_expert activation codes: M0 = buffer + gi * PF_GRP + t * PF_RS with slot
// group gi <= PF_TB - 1 (8 waves: wave >> 2; 4 waves: k < 2) and t = 4 * wq +
// (jj & 3) <= 15; lanes 32..63 fill slot t + 16, 512 bytes on.
static_assert((PF_TB - 1u) * PF_GRP + 15u * PF_RS + DMA16_SPAN <= PF_ACT_BUF, "pf_expert code loads stay in their buffer");
static_assert(DMA16_SPAN == 2u * 512u && 512u == 2u * SF37_QK, "one load = slots t and t + 16, 512 bytes each");
static_assert(PF_RS >= 512u, "a slot row holds a block's 256 fp16 codes");

// ---------------------------------------------------------------------------
// Pair layouts.  Lane half kh of an MFMA holds 32 codes of every 64-group
// (codes 32kh .. 32kh+31) as 16 pairs; pair P feeds MFMA P/4, dword P%4.
// ---------------------------------------------------------------------------
// Q3 (3-bit codes at bit 3c of the lane's 96-bit string).  Window = the
// string shifted right by the window offset; type = where the two codes sit
// in the window: A1 bits 0 / 18, A2 bits 3 / 21, B1 bits 1 / 16, B2 bits 4 / 19.
__constant__ uint8_t q3_lo_c[16] = {0, 1, 2, 3, 4, 5, 12, 13, 14, 15, 16, 22, 23, 24, 25, 26};
__constant__ uint8_t q3_hi_c[16] = {6, 7, 8, 9, 10, 11, 17, 18, 19, 20, 21, 27, 28, 29, 30, 31};
__constant__ uint8_t q3_ty_c[16] = {0, 1, 0, 1, 0, 1, 2, 3, 2, 3, 2, 2, 3, 2, 3, 2};
// mantissa bit of the low / high code of each type (high relative to bit 16)
__host__ __device__ constexpr uint32_t q3_plo(uint32_t ty) { return ty == 0 ? 0u : ty == 1 ? 3u : ty == 2 ? 1u : 4u; }
__host__ __device__ constexpr uint32_t q3_phi(uint32_t ty) { return ty == 0 ? 2u : ty == 1 ? 5u : ty == 2 ? 0u : 3u; }
__host__ __device__ constexpr uint32_t q3_mask(uint32_t ty) {
    return (7u << q3_plo(ty)) | (7u << (16u + q3_phi(ty)));
}
__host__ __device__ constexpr uint32_t pf_exp(uint32_t plo, uint32_t phi) {
    return ((25u - plo) << 10) | ((25u - phi) << 26);
}
__host__ __device__ constexpr uint32_t pf_mul(uint32_t plo, uint32_t phi) {
    return (1u << plo) | (1u << (16u + phi));
}

// ---------------------------------------------------------------------------
// Activation kernel: Q8_K of one (row, 256-block) per wave, then the codes
// in MFMA order as fp16, C per 64-group and d.
// MFMA order of a block: position 64g + 32kh + 8m + e holds the code of
// pair P = 4m + e/2 (low code if e even, high if odd) of lane half kh.
// ---------------------------------------------------------------------------
template <bool Q3>
__device__ __forceinline__ void pf_pos_code(uint32_t pos, uint32_t &code, int32_t &bias) {
    const uint32_t kh = (pos >> 5) & 1u, m = (pos >> 3) & 3u, e = pos & 7u;
    const uint32_t P = 4u * m + (e >> 1), half = e & 1u;
    if (Q3) {
        const uint32_t ty = q3_ty_c[P];
        code = 32u * kh + (half ? q3_hi_c[P] : q3_lo_c[P]);
        bias = (int32_t)(1u << (10u - (half ? q3_phi(ty) : q3_plo(ty)))) + 8;
    } else {
        const uint32_t k = P & 3u, qd = P >> 2;
        code = 32u * kh + 16u * (qd >> 1) + 4u * (qd & 1u) + k + 8u * half;
        bias = (int32_t)(1u << (10u - 2u * k)) + 4;
    }
}

template <bool Q3>
__global__ void __launch_bounds__(256) pf_act_kernel(_Float16 *__restrict__ codes, float *__restrict__ tab,
                                                     const float *__restrict__ x, uint32_t nblk,
                                                     uint32_t n_rows) {
    // each wave owns its LDS row and walks the (row, block) units wave by
    // wave over the grid; nothing is shared between waves
    __shared__ int8_t qs[4][SF37_QK];
    const uint32_t wv = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t units = nblk * n_rows, stride = gridDim.x * 4u;
    // lane produces positions 4*lane .. 4*lane+3, all in group lane/16: their
    // source codes and biases do not depend on the unit
    const uint32_t g = lane >> 4;
    uint32_t code[4];
    int32_t bias[4];
#pragma unroll
    for (uint32_t c = 0; c < 4u; c++) pf_pos_code<Q3>(4u * (lane & 15u) + c, code[c], bias[c]);
    for (uint32_t u = blockIdx.x * 4u + wv; u < units; u += stride) {
        const float *xb = x + (uint64_t)u * SF37_QK + 4u * lane;
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = xb[k];
        int8_t q[4];
        int gs;
        const float d = q8k_codes4(v, q, gs);
        (void)gs;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the previous unit's reads are done
#pragma unroll
        for (int k = 0; k < 4; k++) qs[wv][4u * lane + k] = q[k];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // this unit's codes are in LDS
        __builtin_amdgcn_wave_barrier();
        int32_t s = 0;
        _Float16 h[4];
#pragma unroll
        for (uint32_t c = 0; c < 4u; c++) {
            const int32_t a = qs[wv][64u * g + code[c]];
            h[c] = (_Float16)a;
            s += bias[c] * a;
        }
        s = wave_sum_i32_width(s, 16);
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        const h4 hv = {h[0], h[1], h[2], h[3]};
        *(h4 *)(codes + (uint64_t)u * SF37_QK + 4u * lane) = hv;
        float *tb = tab + (uint64_t)u * PF_TAB;
        if ((lane & 15u) == 0u) tb[g] = (float)(-s);
        if (lane == 0u) tb[4] = d;
    }
}

// ---------------------------------------------------------------------------
// Tile list: every group split into tiles of <= PF_T pairs.
// tiles[0] = count; tile t at uint4 index 1 + t = {expert, first pair, count, 0}.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(1024) pf_tiles_kernel(uint32_t *__restrict__ tiles,
                                                        const uint32_t *__restrict__ ginfo,
                                                        uint32_t max_groups) {
    __shared__ uint32_t wsum[16];
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
    const uint32_t ng = ginfo[0];
    uint32_t base = 0;
    for (uint32_t g0 = 0; g0 < ng; g0 += 1024u) {
        const uint32_t g = g0 + tid;
        uint32_t nt = 0, p0 = 0, cnt = 0;
        if (g < ng) {
            p0 = ginfo[1 + g];
            cnt = ginfo[2 + g] - p0;
            nt = (cnt + PF_T - 1u) / PF_T;
        }
        uint32_t sc = nt;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t a = __shfl_up(sc, o, 64);
            if (lane >= (uint32_t)o) sc += a;
        }
        if (lane == 63u) wsum[wave] = sc;
        __syncthreads();
        uint32_t before = base, all = 0;
        for (uint32_t w = 0; w < 16u; w++) {
            if (w < wave) before += wsum[w];
            all += wsum[w];
        }
        const uint32_t first = before + sc - nt;
        if (g < ng) {
            const uint32_t e = ginfo[2 + max_groups + g];
            for (uint32_t k = 0; k < nt; k++) {
                const uint32_t c = cnt - k * PF_T < PF_T ? cnt - k * PF_T : PF_T;
                ((uint4 *)tiles)[1 + first + k] = make_uint4(e, p0 + k * PF_T, c, 0u);
            }
        }
        base += all;
        __syncthreads();
    }
    if (tid == 0) tiles[0] = base;
}

// ---------------------------------------------------------------------------
// Tables in dispatch order: tabs[(b * 5 + a) * stride + s] = tab[row(s)][b][a]
// for sorted position s (row = pair / div: the token for x, the pair for the
// mid), a = C0..C3, d.  A tile's entries are then contiguous.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) pf_tab_sort_kernel(float *__restrict__ tabs, const float *__restrict__ tab,
                                                          const uint32_t *__restrict__ sorted, uint32_t n_pairs,
                                                          uint32_t nblk, uint32_t div, uint32_t stride) {
    const uint32_t s = blockIdx.x * 256u + threadIdx.x, b = blockIdx.y;
    if (s >= n_pairs) return;
    const float *t = tab + ((uint64_t)(sorted[s] / div) * nblk + b) * PF_TAB;
    const float4 c = *(const float4 *)t;
    float *o = tabs + (uint64_t)b * 5u * stride + s;
    o[0] = c.x;
    o[(uint64_t)stride] = c.y;
    o[2ull * stride] = c.z;
    o[3ull * stride] = c.w;
    o[4ull * stride] = t[4];
}

// ---------------------------------------------------------------------------
// LDS direct loads (global -> LDS, no registers).  Issued through inline asm
// so the compiler does not wait for them before unrelated LDS reads; the
// kernel waits with s_waitcnt vmcnt(0) + barrier before reading the buffer.
// Lane i of a dwordx4 load writes LDS bytes [m0 + 16 i, m0 + 16 i + 16);
// one wait state separates the M0 write from the load.  m0 cannot be named
// as a clobber (the compiler reserves it and drops such a clobber), so these
// sequences rely on no compiler-generated code of these kernels reading m0:
// in the gfx950 assembly of this file every m0 access is one of these
// s_mov_b32 writes (no movrel, gpr-index or sendmsg use).
// ---------------------------------------------------------------------------
// sbase must be wave-uniform; it is moved to SGPRs with readfirstlane.
__device__ __forceinline__ uint64_t sgpr_ptr(const void *p) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ void lds_dma16(uint32_t lds, uint32_t voff, const void *sbase) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(__builtin_amdgcn_readfirstlane(lds)),
                 "v"(voff), "s"(sgpr_ptr(sbase))
                 : "memory");
}
__device__ __forceinline__ void lds_dma4(uint32_t lds, uint32_t voff, const void *sbase) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2" ::"s"(__builtin_amdgcn_readfirstlane(lds)),
                 "v"(voff), "s"(sgpr_ptr(sbase))
                 : "memory");
}
__device__ __forceinline__ void wait_vm0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// All but the newest PF_DMA_PER_BLOCK vector-memory operations of the wave
// done: the activation loads issued for the block after next stay in flight
// (8-wave workgroups, three buffers).
constexpr int PF_DMA_PER_BLOCK = 5;   // 4 code rows + 1 table row per wave and block
static_assert(PF_DMA_PER_BLOCK == 5, "the count in wait_vm_keep_next");
__device__ __forceinline__ void wait_vm_keep_next() { asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); }

// After wait_vm0, mark a block's weight words as just defined: the compiler
// then knows no load is pending on them and does not place its own
// s_waitcnt vmcnt inside the compute (which would also wait for the next
// block's LDS direct loads, issued earlier in program order).
struct q3_raw;
struct q2_raw;

__device__ __forceinline__ uint32_t lds_addr(const void *p) { return (uint32_t)(uintptr_t)p; }

struct pf_params {
    float *mid, *gate_out, *up_out, *down_pair;
    const uint8_t *w0, *w1;        // gate / up (Q3) or down (Q2)
    const _Float16 *act;           // [rows][nblk * 256] codes in MFMA order
    const float *tab;              // [nblk][5][tab_stride] tables in dispatch order
    const uint32_t *tiles;
    const uint32_t *sorted;
    const float *weights;
    uint32_t topk, nblk, out_rows, n_rt, tab_stride;
    float clamp;
};

// Weight bytes of one lane for one block.
struct q3_raw {
    uint32_t h[4];      // header dwords (scales, zero points)
    uint32_t w[4][4];   // per group: 16 aligned bytes holding the lane's 12
};
struct q2_raw {
    uint32_t h[3];
    uint32_t w[4][2];
};


__device__ __forceinline__ void raw_ready(q3_raw &r) {
    asm volatile("" : "+v"(r.h[0]), "+v"(r.h[1]), "+v"(r.h[2]), "+v"(r.h[3]), "+v"(r.w[0][0]), "+v"(r.w[0][1]),
                 "+v"(r.w[0][2]), "+v"(r.w[0][3]), "+v"(r.w[1][0]), "+v"(r.w[1][1]), "+v"(r.w[1][2]),
                 "+v"(r.w[1][3]), "+v"(r.w[2][0]), "+v"(r.w[2][1]), "+v"(r.w[2][2]), "+v"(r.w[2][3]),
                 "+v"(r.w[3][0]), "+v"(r.w[3][1]), "+v"(r.w[3][2]), "+v"(r.w[3][3]));
}

typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x3a __attribute__((ext_vector_type(3), aligned(4)));
typedef uint32_t u32x2a __attribute__((ext_vector_type(2), aligned(4)));

// Q3 words as dword loads (no register tuples): the words go straight into
// the registers the loop carries them in, so no copy waits for the data.
// (Contiguous half-block loads with lane swaps, as the Q2 blocks below,
// measured 1.5 % slower here: twelve swaps per block cost more VALU than
// the sixteen fewer loads save in this VALU-bound kernel.)
__device__ __forceinline__ void q3_load(q3_raw &r, const uint8_t *hp, const uint8_t *pp) {
    const uint32_t *h = (const uint32_t *)hp;
#pragma unroll
    for (int i = 0; i < 4; i++) r.h[i] = h[i];
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const uint32_t *q = (const uint32_t *)(pp + 24 * g);
#pragma unroll
        for (int i = 0; i < 4; i++) r.w[g][i] = q[i];
    }
}


// What a lane loads of a Q2 block (21 dwords): dwords 8 kh .. 8 kh + 10,
// contiguous (three loads instead of eleven); pf_words then trades what each
// half needs from the other with v_permlane32_swap (lanes l and l + 32 hold
// the same row).
struct q2_half {
    uint32_t w[11];
};
__device__ __forceinline__ void raw_ready(q2_half &r) {
    asm volatile("" : "+v"(r.w[0]), "+v"(r.w[1]), "+v"(r.w[2]), "+v"(r.w[3]), "+v"(r.w[4]), "+v"(r.w[5]),
                 "+v"(r.w[6]), "+v"(r.w[7]), "+v"(r.w[8]), "+v"(r.w[9]), "+v"(r.w[10]));
}
__device__ __forceinline__ void q2_load_half(q2_half &r, const uint8_t *bp, uint32_t kh) {
    const uint32_t *q = (const uint32_t *)bp + 8u * kh;
#pragma unroll
    for (int i = 0; i < 11; i++) r.w[i] = q[i];
}
// q2_raw of both halves: the header dwords 0..2 and group g's dwords
// 3 + 4 g + 2 kh, +1.  permlane32_swap(A, B) gives [A of lanes 0-31, B of
// lanes 0-31] and [A of lanes 32-63, B of lanes 32-63]; with A, B = loaded
// dwords (3, 5), (4, 6), (7, 9), (8, 10) the first is a word of group 0 or 1
// for both halves, the second the same word of group 2 or 3 (8 dwords on);
// a swap of dword j with itself hands both halves header dword j.
__device__ __forceinline__ q2_raw pf_words(const q2_half &h) {
    q2_raw r;
#pragma unroll
    for (int j = 0; j < 3; j++) r.h[j] = __builtin_amdgcn_permlane32_swap(h.w[j], h.w[j], false, false)[0];
#pragma unroll
    for (int g = 0; g < 2; g++) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const auto v = __builtin_amdgcn_permlane32_swap(h.w[3 + 4 * g + i], h.w[5 + 4 * g + i], false, false);
            r.w[g][i] = v[0];
            r.w[g + 2][i] = v[1];
        }
    }
    return r;
}
__device__ __forceinline__ const q3_raw &pf_words(const q3_raw &r) { return r; }

// 32 bits of the lane's string starting at bit SH + o of the loaded words.
template <int SH, int O>
__device__ __forceinline__ uint32_t q3_win(const uint32_t *w) {
    constexpr int a = SH + O, k = a >> 5, s = a & 31;
    if constexpr (s == 0) return w[k];
    else return align_bits(w[k + 1], w[k], (uint32_t)s);
}

// f16 scale of group g, zero point of group g from the header bits at SH.
template <int SH>
__device__ __forceinline__ float hdr_scale(const uint32_t *h, int g) {
    const int a = SH + 16 * g;
    return sf37_f16(h[a >> 5] >> (a & 31));
}
template <int SH>
__device__ __forceinline__ uint32_t hdr_zp(const uint32_t *h, int g) {
    const int a = SH + 64 + 8 * g;
    return (h[a >> 5] >> (a & 31)) & 0xffu;
}

// Q3 / Q2 dequantisation of part (0: pair words 0..7, 1: words 8..15) of group g.
template <bool Q3, int SH, int PART, typename RAW>
__device__ __forceinline__ void pf_dequant(const RAW &r, int g, uint32_t out[16]) {
    if constexpr (Q3) {
        const uint32_t k = 8u - (hdr_zp<SH>(r.h, g) & 7u);
        const uint32_t *w = r.w[g];
        constexpr uint32_t mA1 = q3_mask(0), mA2 = q3_mask(1), mB1 = q3_mask(2), mB2 = q3_mask(3);
        const uint32_t cB1 = pf_exp(1, 0) + k * pf_mul(1, 0), cB2 = pf_exp(4, 3) + k * pf_mul(4, 3);
        uint32_t x;
        if constexpr (PART == 0) {
            const uint32_t cA1 = pf_exp(0, 2) + k * pf_mul(0, 2), cA2 = pf_exp(3, 5) + k * pf_mul(3, 5);
            x = q3_win<SH, 0>(w);  out[0] = (x & mA1) + cA1;  out[1] = (x & mA2) + cA2;
            x = q3_win<SH, 6>(w);  out[2] = (x & mA1) + cA1;  out[3] = (x & mA2) + cA2;
            x = q3_win<SH, 12>(w); out[4] = (x & mA1) + cA1;  out[5] = (x & mA2) + cA2;
            x = q3_win<SH, 35>(w); out[6] = (x & mB1) + cB1;  out[7] = (x & mB2) + cB2;
        } else {
            x = q3_win<SH, 41>(w); out[8] = (x & mB1) + cB1;  out[9] = (x & mB2) + cB2;
            x = q3_win<SH, 47>(w); out[10] = (x & mB1) + cB1;
            x = q3_win<SH, 65>(w); out[11] = (x & mB1) + cB1; out[12] = (x & mB2) + cB2;
            x = q3_win<SH, 71>(w); out[13] = (x & mB1) + cB1; out[14] = (x & mB2) + cB2;
            x = q3_win<SH, 77>(w); out[15] = (x & mB1) + cB1;
        }
    } else {
        const uint32_t k = 4u - (hdr_zp<0>(r.h, g) & 3u);
        const uint32_t u = r.w[g][PART];
#pragma unroll
        for (uint32_t h = 0; h < 2u; h++) {
            const uint32_t x = h ? (u >> 8) : u;
#pragma unroll
            for (uint32_t j = 0; j < 4u; j++)
                out[8 * PART + 4u * h + j] =
                    (x & (0x00030003u << (2u * j))) + pf_exp(2u * j, 2u * j) + k * pf_mul(2u * j, 2u * j);
        }
    }
}

// One 256-block of the tile.  Chains c = (group g, token block i), 4*NTB of
// them, each = 4 MFMAs on accumulator D = C(g, i).  Stage c calls pre(c)
// (a slice of the next block's global loads, so a stalled memory issue
// overlaps MFMAs already in flight), issues the LDS loads of chain c+1,
// part of the next group's dequantisation, the MFMAs of chain c and the
// epilogue blk = fma(s_g, D, blk) of chain c-1; stages are fenced so the
// compiler interleaves within a stage only.  Then acc = fma(d, blk, acc)
// per token block.
template <bool Q3, int SH, int NTB, typename RAW, typename PRE>
__device__ __forceinline__ void pf_block(const RAW &r, const uint8_t *act_lds, const float *cd_lds,
                                         uint32_t kh, uint32_t col, float (*acc)[16], f16v blk[PF_TB],
                                         PRE &&pre) {
    constexpr int NC = 4 * NTB;
    const uint8_t *a_lane = act_lds + (col & 15u) * PF_RS + (col >> 4) * 512u + 64u * kh;
    const float *c_lane = cd_lds + 4u * kh;
    uint32_t bw[2][16];
    float s[4];
#pragma unroll
    for (int g = 0; g < 4; g++) s[g] = hdr_scale<Q3 ? SH : 0>(r.h, g);
    pf_dequant<Q3, SH, 0>(r, 0, bw[0]);
    pf_dequant<Q3, SH, 1>(r, 0, bw[0]);
    f16v D[3];
    h8 A[2][4];
    auto load = [&](int c, f16v &d, h8 *a) {
        const int g = c / NTB, i = c % NTB;
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            const float4 v = *(const float4 *)(c_lane + g * PF_T + 32 * i + 8 * jj);
            d[4 * jj] = v.x; d[4 * jj + 1] = v.y; d[4 * jj + 2] = v.z; d[4 * jj + 3] = v.w;
        }
#pragma unroll
        for (int m = 0; m < 4; m++) a[m] = *(const h8 *)(a_lane + i * PF_GRP + (8 * g + m) * 16);
    };
    load(0, D[0], A[0]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int g = c / NTB, i = c % NTB;
        pre(c, NC);
        if (c + 1 < NC) load(c + 1, D[(c + 1) % 3], A[(c + 1) & 1]);
        if (g < 3) {
            constexpr int P0 = NTB >= 3 ? 1 : 0, P1 = NTB >= 3 ? 2 : NTB - 1;
            if (i == P0) pf_dequant<Q3, SH, 0>(r, g + 1, bw[(g + 1) & 1]);
            if (i == P1) pf_dequant<Q3, SH, 1>(r, g + 1, bw[(g + 1) & 1]);
        }
        {
            const uint32_t *bb = bw[g & 1];
#pragma unroll
            for (int m = 0; m < 4; m++) {
                typedef uint32_t u4 __attribute__((ext_vector_type(4)));
                const u4 t = {bb[4 * m], bb[4 * m + 1], bb[4 * m + 2], bb[4 * m + 3]};
                D[c % 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[c & 1][m], __builtin_bit_cast(h8, t), D[c % 3], 0, 0, 0);
            }
        }
        if (c > 0) {
            const int gp = (c - 1) / NTB, ip = (c - 1) % NTB;
#pragma unroll
            for (int r2 = 0; r2 < 16; r2++)
                blk[ip][r2] = __builtin_fmaf(s[gp], D[(c - 1) % 3][r2], gp == 0 ? 0.0f : blk[ip][r2]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int r2 = 0; r2 < 16; r2++)
        blk[NTB - 1][r2] = __builtin_fmaf(s[3], D[(NC - 1) % 3][r2], blk[NTB - 1][r2]);
#pragma unroll
    for (int i = 0; i < NTB; i++) {
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            const float4 d = *(const float4 *)(c_lane + 4 * PF_T + 32 * i + 8 * jj);
            acc[i][4 * jj] = __builtin_fmaf(d.x, blk[i][4 * jj], acc[i][4 * jj]);
            acc[i][4 * jj + 1] = __builtin_fmaf(d.y, blk[i][4 * jj + 1], acc[i][4 * jj + 1]);
            acc[i][4 * jj + 2] = __builtin_fmaf(d.z, blk[i][4 * jj + 2], acc[i][4 * jj + 2]);
            acc[i][4 * jj + 3] = __builtin_fmaf(d.w, blk[i][4 * jj + 3], acc[i][4 * jj + 3]);
        }
    }
}

template <bool Q3> using pf_raw_t = typename std::conditional<Q3, q3_raw, q2_half>::type;

// One tile's view for the routed kernels: its expert, pairs and weight row,
// and the per-lane direct-load offsets of its activation rows.
template <bool Q3>
struct pf_item {
    uint32_t e, p0, cnt, ntb;
    const uint8_t *wrow;
    uint32_t wcol;
    uint32_t voff[pf_cfg<Q3>::NW == 8u ? 4 : 1];
    uint32_t rowoff_c[pf_cfg<Q3>::NW == 8u ? 1 : 2];
};

// A block's weight words into r (even blocks start dword-aligned, odd Q3
// blocks 2 bytes in).
template <bool Q3>
__device__ __forceinline__ void pf_wload(pf_raw_t<Q3> &r, const uint8_t *wrow, uint32_t bn, uint32_t kh) {
    if constexpr (Q3) {
        const uint32_t o = SF37_Q3_BYTES * bn;
        q3_load(r, wrow + (o & ~3u), wrow + ((o + 12u + 12u * kh) & ~3u));
    } else {
        q2_load_half(r, wrow + (uint64_t)SF37_Q2_BYTES * bn, kh);
    }
}

// The block loop for NTB 32-pair blocks (the tile's pair count rounded up).
// On entry block 0's weights are loading into ra and its activation rows
// (with NBUF = 3, block 1's too) are issued; on exit every load is done.
//
// Pipeline: a block's weight words (registers) are loaded one block
// ahead.  Three activation buffers (8 waves): the activation rows and
// tables of block b+2 are loaded during block b, spread over its stages,
// and the top of block b+1 waits for all but those newest
// PF_DMA_PER_BLOCK loads.  Two buffers (4 waves): those of block b+1 are
// issued at the start of block b, and the top of block b+1 waits for
// every load.  Past the last block the loads repeat block nblk-1 (its
// buffer then receives the same bytes again; uniform code, no branch
// inside the stages); the final wait keeps no load in flight at the end
// of the workgroup.
template <bool Q3, int NTB, typename ISSUE>
__device__ __forceinline__ void pf_loop(const pf_params &p, const uint8_t *wrow, ISSUE &&issue_act,
                                        uint8_t (*s_act)[PF_ACT_BUF], float (*s_cd)[PF_CD_ROWS * PF_T],
                                        uint32_t kh, uint32_t col, pf_raw_t<Q3> &ra, float (*acc)[16]) {
    const uint32_t nblk = p.nblk;
    f16v blk[PF_TB];
#pragma unroll
    for (int i = 0; i < NTB; i++)
#pragma unroll
        for (int r2 = 0; r2 < 16; r2++) acc[i][r2] = 0.0f;
    constexpr uint32_t NBUF = pf_cfg<Q3>::NBUF;
    const uint32_t last = nblk - 1u;
    auto clampb = [&](uint32_t x) { return x < nblk ? x : last; };
    auto top = [&]() {
        if constexpr (NBUF == 3u) wait_vm_keep_next();
        else wait_vm0();
    };
    pf_raw_t<Q3> rb;
    // the block's loads: weights of bn into r, activations of ba
    auto pre = [&](pf_raw_t<Q3> &r, uint32_t bn, uint32_t ba, int c, int nc) {
        if (c == 0) pf_wload<Q3>(r, wrow, bn, kh);
        if constexpr (NBUF == 3u) issue_act(ba, c, nc);
        else if (c == 0) issue_act(ba, 0, 1);
    };
    constexpr int SH2 = Q3 ? 16 : 0;   // bit offset of an odd block's string in its words
    for (uint32_t b = 0; b < nblk; b += 2u) {
        top();
        raw_ready(ra);
        __syncthreads();
        const uint32_t b1 = clampb(b + 1u), b2 = clampb(b + 2u), b3 = clampb(b + 3u);
        pf_block<Q3, 0, NTB>(pf_words(ra), s_act[b % NBUF], s_cd[b % NBUF], kh, col, acc, blk,
                             [&](int c, int nc) { pre(rb, b1, NBUF == 3u ? b2 : b1, c, nc); });
        if (b + 1u < nblk) {
            top();
            raw_ready(rb);
            __syncthreads();
            pf_block<Q3, SH2, NTB>(pf_words(rb), s_act[(b + 1u) % NBUF], s_cd[(b + 1u) % NBUF], kh, col, acc, blk,
                                   [&](int c, int nc) { pre(ra, b2, NBUF == 3u ? b3 : b2, c, nc); });
        }
    }
    wait_vm0();
}

// The tile's outputs.  D layout: lane holds column col, tokens
// 8*(r/4) + 4*kh + r%4.  Gate/up: mid = ((g*sig(g))*u)*w per pair; down:
// the per-pair rows.
template <bool Q3, int NTB>
__device__ __forceinline__ void pf_epilogue(const pf_params &p, const float (*acc)[16], const uint32_t *s_pair,
                                            const float *s_w, const uint64_t *s_tab, uint32_t kh, uint32_t col,
                                            uint32_t wcol, uint32_t cnt) {
#pragma unroll
    for (uint32_t i = 0; i < (uint32_t)NTB; i++) {
        if constexpr (Q3) {
            // lanes col and col ^ 16 hold the gate and up rows of one mid row:
            // after swapping values the gate lane forms the SwiGLU of tokens
            // r2 = k and the up lane of r2 = k + 8, so every lane takes half
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float va = acc[i][k], vb = acc[i][k + 8];
                const float oa = __shfl_xor(va, 16, 64), ob = __shfl_xor(vb, 16, 64);
                const bool up_lane = col >= 16u;
                const int r2 = up_lane ? k + 8 : k;
                const float g = up_lane ? ob : va, u = up_lane ? vb : oa;
                const uint32_t tl = 32u * i + 8u * ((uint32_t)r2 >> 2) + 4u * kh + ((uint32_t)r2 & 3u);
                if (tl < cnt) {
                    const uint64_t at = (uint64_t)s_pair[tl] * p.out_rows + wcol;
                    p.mid[at] = sf37_swiglu_mid_t(g, u, s_w[tl], p.clamp, s_tab);
                    if (p.gate_out) p.gate_out[at] = g;
                    if (p.up_out) p.up_out[at] = u;
                }
            }
        } else {
#pragma unroll
            for (int r2 = 0; r2 < 16; r2++) {
                const uint32_t tl = 32u * i + 8u * (r2 >> 2) + 4u * kh + (r2 & 3);
                if (tl < cnt) p.down_pair[(uint64_t)s_pair[tl] * p.out_rows + wcol] = acc[i][r2];
            }
        }
    }
}

// Gate/up (Q3 = true): row tile = 64 F rows, wave w has gate rows
// rt*64 + 16w + c and up rows (c < 16: gate, else up) as its 32 columns;
// epilogue mid = ((g*sig(g))*u)*w per pair.  Down (Q3 = false): row tile =
// 128 output rows, 32 per wave; epilogue down_pair[pair][row].  One item
// (tile, row tile) per workgroup: tiles interleaved over the XCDs, a tile's
// row tiles consecutive on one.  (A persistent form, each workgroup taking
// every G-th item and issuing the next item's first loads before the
// current item's epilogue, measured slower: down 652 -> 677 us at config 3
// with 40 more VGPRs; gate/up did not fit its registers.)
template <bool Q3>
__global__ void __launch_bounds__(pf_cfg<Q3>::NW * 64, Q3 ? 1 : 2) pf_expert_kernel(pf_params p) {
    constexpr uint32_t NW = pf_cfg<Q3>::NW, NBUF = pf_cfg<Q3>::NBUF;
    __shared__ __align__(16) uint8_t s_act[NBUF][PF_ACT_BUF];
    __shared__ __align__(16) float s_cd[NBUF][PF_CD_ROWS * PF_T];
    __shared__ uint32_t s_pair[PF_T];
    __shared__ float s_w[PF_T];
    __shared__ uint64_t s_tab[Q3 ? 32 : 1];    // the exp table of the SwiGLU epilogue
    const uint32_t tid = threadIdx.x, lane = tid & 63u, kh = lane >> 5, col = lane & 31u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nblk = p.nblk;
    // activation rows: tile slot `lane` for the tables; slot 32*gi + lane%32
    // for the codes (pad slots repeat the last pair).  8 waves: wave 4*gi + wq
    // copies slot group gi; 4 waves: wave wq copies both groups.
    constexpr uint32_t NG = NW == 8u ? 1u : 2u;      // slot groups a wave copies
    constexpr int NJ = 4 * (int)NG;
    const uint32_t wq = wave & 3u;
    const uint32_t act_l = lds_addr(&s_act[0][0]), cd_l = lds_addr(&s_cd[0][0]);
    const uint32_t blk_bytes = Q3 ? SF37_Q3_BYTES : SF37_Q2_BYTES;
    const uint64_t row_bytes = (uint64_t)nblk * blk_bytes;
    // codes: a wave loads slot pairs (t, t + 16), t = 4q .. 4q+3 of its slot
    // group(s): lanes 0..31 read slot t's 512-byte row, lanes 32..63 slot
    // t + 16's.  Each load's per-lane byte offset within a block's codes is
    // the same for every block: the 8-wave kernel forms its four once
    // (measured 1-3 % faster); the 4-wave kernel re-forms its eight per
    // block (eight more VGPRs measured 2 % slower there)
    auto lane_off = [&](const pf_item<Q3> &it, int jj) -> uint32_t {
        const uint32_t k = (uint32_t)jj >> 2, t = 4u * wq + ((uint32_t)jj & 3u);
        const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)it.rowoff_c[k], (int)t);
        const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)it.rowoff_c[k], (int)t + 16);
        return (kh ? r1 : r0) + 16u * col;
    };
    // the workgroup's item (tile, row tile), its pairs and routing weights
    // in s_pair / s_w
    pf_item<Q3> it;
    {
        const uint32_t idx = blockIdx.x, xcd = idx & 7u, slot = idx >> 3;
        const uint32_t t = xcd + 8u * (slot / p.n_rt), rt = slot % p.n_rt;
        if (t >= p.tiles[0]) return;
        const uint4 ti = ((const uint4 *)p.tiles)[1 + t];
        it.e = ti.x;
        it.p0 = ti.y;
        it.cnt = ti.z;
        it.ntb = (it.cnt + 31u) / 32u;
        if (tid < PF_T) {
            const uint32_t pr = p.sorted[it.p0 + (tid < it.cnt ? tid : it.cnt - 1u)];
            s_pair[tid] = pr;
            if (Q3) s_w[tid] = p.weights[pr];
        }
#pragma unroll
        for (uint32_t g = 0; g < NG; g++) {
            const uint32_t gi = NW == 8u ? wave >> 2 : g;
            const uint32_t sl = 32u * gi + (lane & 31u);
            const uint32_t pr = p.sorted[it.p0 + (sl < it.cnt ? sl : it.cnt - 1u)];
            it.rowoff_c[g] = (Q3 ? pr / p.topk : pr) * nblk * (SF37_QK * 2u);
        }
        if constexpr (NW == 8u) {
#pragma unroll
            for (int jj = 0; jj < NJ; jj++) it.voff[jj] = lane_off(it, jj);
        }
        // this lane's weight row
        it.wcol = Q3 ? rt * PF_GU_R + 16u * wave + (col & 15u) : rt * PF_DN_R + 32u * wave + col;
        it.wrow = (Q3 && col >= 16u ? p.w1 : p.w0) + ((uint64_t)it.e * p.out_rows + it.wcol) * row_bytes;
    }
    if (Q3) sf37_stage_exp_tab(s_tab);          // read after the block loop's barriers
    // slice `part` of `nparts` (compile-time after inlining) of block b's
    // activation loads
    auto issue_act = [&](uint32_t b, int part, int nparts) {
        const uint32_t bf = b % NBUF;
        const uint8_t *cb = (const uint8_t *)p.act + (uint64_t)b * (SF37_QK * 2u);
        const int j0 = NJ * part / nparts, j1 = NJ * (part + 1) / nparts;
#pragma unroll
        for (int jj = j0; jj < j1; jj++) {
            const uint32_t k = (uint32_t)jj >> 2, gi = NW == 8u ? wave >> 2 : k;
            const uint32_t t = 4u * wq + ((uint32_t)jj & 3u);
            uint32_t vo;
            if constexpr (NW == 8u) vo = it.voff[jj];
            else vo = lane_off(it, jj);
            lds_dma16(act_l + bf * PF_ACT_BUF + gi * PF_GRP + t * PF_RS, vo, cb);
        }
        if (part == 0) {   // tables of all slots: row a = C_a (a < 4) or d (a = 4).  8 waves:
                           // wave a < 5 loads row a, waves 5..7 row 4 again; 4 waves: wave w
                           // loads rows w and 4 (the same bytes from every wave; no branch)
#pragma unroll
            for (uint32_t k = 0; k < (NW == 8u ? 1u : 2u); k++) {
                const uint32_t a = NW == 8u ? (wave < 5u ? wave : 4u) : (k ? 4u : wave);
                const float *tb = p.tab + ((uint64_t)b * 5u + a) * p.tab_stride + it.p0;
                lds_dma4(cd_l + bf * (PF_CD_ROWS * PF_T * 4u) + (NW == 8u ? wave : a) * PF_T * 4u, 4u * lane, tb);
            }
        }
    };
    // the first loads: block 0's weights, its activation rows (and block 1's
    // with three buffers)
    pf_raw_t<Q3> ra;
    issue_act(0, 0, 1);
    pf_wload<Q3>(ra, it.wrow, 0, kh);
    if constexpr (NBUF == 3u) issue_act(nblk > 1u ? 1u : 0u, 0, 1);
    float acc[2][16];
    if (it.ntb == 1) {
        pf_loop<Q3, 1>(p, it.wrow, issue_act, s_act, s_cd, kh, col, ra, acc);
        pf_epilogue<Q3, 1>(p, acc, s_pair, s_w, s_tab, kh, col, it.wcol, it.cnt);
    } else {
        pf_loop<Q3, 2>(p, it.wrow, issue_act, s_act, s_cd, kh, col, ra, acc);
        pf_epilogue<Q3, 2>(p, acc, s_pair, s_w, s_tab, kh, col, it.wcol, it.cnt);
    }
}

// ---------------------------------------------------------------------------
// Shared expert (Q8_0, every token) on the int8 matrix cores.
//
// Canonical order of sf37_ops.c:92-108: acc = acc + ((float)isum_b * ws_b) * xs_b
// per 32-block in block order.  One v_mfma_i32_32x32x32_i8 per (32-block,
// 32-token block) forms isum_b exactly from the Q8_0 weight codes, read in
// place from the tensor (no repacked copy), and the Q8_0 activation codes.
// Its accumulator starts at the bits of SH_MAGIC = 1.5 * 2^23, so the int32
// result read as a float is F = SH_MAGIC + isum_b exactly (|isum_b| <=
// 32 * 127 * 128 < 2^22), and fma(F, ws_b, -SH_MAGIC * ws_b) is the exact
// isum_b * ws_b (the second term is exact: 2 * 11 significant bits) rounded
// once, the CPU's (float)isum * w_scale.  The epilogue is then the CPU's
// three float operations per output and block.
//
// Layouts.  Activations: Q8_0 codes of each token in natural order (int8,
// nb * 32 bytes per token) and a float scale per (token, block), bit-exact
// with sf37_ops.c:57-90.  A workgroup stages a chunk of SH_CB blocks of its
// 64 tokens in LDS: token row r holds 2 * SH_CB 16-byte pieces (block jj,
// half kh = piece 2 jj + kh), piece q stored at slot q ^ (r & 7), so the
// 8 rows a read of 8 lanes touches land on distinct banks.  MFMA operands:
// lane (row or column l % 32, half kh = l / 32) holds the 16 codes
// 16 kh .. 16 kh + 15 of a block, for activations and weights alike.
// ---------------------------------------------------------------------------
constexpr uint32_t SH_T = 64;                  // tokens per tile
constexpr uint32_t SH_CB = 4;                  // Q8_0 blocks per K chunk
constexpr uint32_t SH_RS = SH_CB * 32u;        // LDS bytes per token row of a chunk (int8 codes)
constexpr uint32_t SH_BUF = SH_T * SH_RS;      // one chunk buffer
constexpr float SH_MAGIC = 12582912.0f;        // 1.5 * 2^23
constexpr int32_t SH_MAGIC_BITS = 0x4B400000;
// sh_gemm direct loads (dwordx4): load L of a chunk fills token rows
// 8 L .. 8 L + 7 (1 KiB, contiguous), L < SH_T / 8, two per wave (4 waves);
// activation scales (dword): row `wave` of SH_T floats.
static_assert(SH_RS == 128u && DMA16_SPAN == 8u * SH_RS && SH_T / 8u == 2u * 4u,
              "sh_gemm code loads: 8 rows each, two per wave, inside the buffer");
static_assert(7u * DMA16_SPAN + DMA16_SPAN <= SH_BUF, "sh_gemm code loads stay in their buffer");
static_assert(SH_T * 4u == DMA4_SPAN && 4u <= SH_CB, "sh_gemm scale rows stay in their buffer");

// Q8_0 activations (arithmetic of q8_0_quantize_kernel, k_q8_0.hip): eight
// lanes per 32-block, four consecutive values per lane, whose codes are one
// dword store; the scale as a float.
__global__ void __launch_bounds__(256) sh_act_kernel(int8_t *__restrict__ a8, float *__restrict__ xs,
                                                     const float *__restrict__ x, uint32_t nb, uint64_t n_tok) {
    const uint64_t gid = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    const uint64_t blk = gid >> 3;
    const uint32_t j = (uint32_t)gid & 7u;
    const bool live = blk < nb * n_tok;
    const uint64_t u = live ? blk : 0u;
    const float4 v = *(const float4 *)(x + u * 32u + 4u * j);
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
    for (int off = 4; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 8));
    uint32_t q = 0;
    float d = 0.0f;
    if (amax != 0.0f) {
        d = amax / 127.0f;
        const float iscale = 1.0f / d;
        const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int c = (int)fminf(fmaxf(__builtin_rintf(iscale * vv[k]), -128.0f), 127.0f);
            q |= ((uint32_t)c & 0xffu) << (8 * k);
        }
    }
    if (!live) return;
    *(uint32_t *)(a8 + u * 32u + 4u * j) = q;
    if (j == 0u) xs[u] = d;
}

struct sh_params {
    float *out0;                   // gate/up: mid (SwiGLU) [tok][rows]; down: out [tok][rows]
    const uint8_t *w0, *w1;        // Q8_0 gate, up (or down) [rows][nb blocks]
    const int8_t *act;             // [tok][nb * 32]
    const float *xs;               // [tok][nb]
    uint32_t n_tok, nb, rows, n_ct, n_tt;
    float clamp;
};

// The lane's weight words of one K chunk: per block its 16 codes (half kh)
// from the dwords around them (block jj of a chunk starts at byte 34 jj of
// the chunk, so even blocks' codes sit 2 bytes into a dword and odd blocks'
// on a dword boundary), and the dword holding the f16 scale.
struct sh_raw {
    uint32_t c[18];                // 5 + 4 + 5 + 4 code dwords
    uint32_t s[4];
};

// What a lane loads of a K chunk: its half of the row's 136 bytes, dwords
// 17 kh .. 17 kh + 16, contiguous (five loads instead of one per block
// piece; lanes l and l + 32 hold the same row).
struct sh_half {
    uint32_t w[17];
};

__device__ __forceinline__ void sh_ready(sh_half &h) {
    asm volatile("" : "+v"(h.w[0]), "+v"(h.w[1]), "+v"(h.w[2]), "+v"(h.w[3]), "+v"(h.w[4]), "+v"(h.w[5]),
                 "+v"(h.w[6]), "+v"(h.w[7]), "+v"(h.w[8]));
    asm volatile("" : "+v"(h.w[9]), "+v"(h.w[10]), "+v"(h.w[11]), "+v"(h.w[12]), "+v"(h.w[13]), "+v"(h.w[14]),
                 "+v"(h.w[15]), "+v"(h.w[16]));
}

// dword offsets (within the chunk) of block jj's first code dword for half
// kh = 0, and of the dword holding its scale; the scale is that dword's high
// half for odd jj
__host__ __device__ constexpr uint32_t sh_code_dw(uint32_t jj) { return (34u * jj + 2u) / 4u; }
__host__ __device__ constexpr uint32_t sh_scale_dw(uint32_t jj) { return (34u * jj) / 4u; }
// first of block jj's code dwords in sh_raw::c (5 for even blocks, 4 for odd)
__host__ __device__ constexpr uint32_t sh_code_reg(uint32_t jj) { return (9u * jj + 1u) / 2u; }
static_assert(sh_code_dw(0) == 0 && sh_code_dw(1) == 9 && sh_code_dw(2) == 17 && sh_code_dw(3) == 26 &&
                  sh_scale_dw(1) == 8 && sh_scale_dw(3) == 25 && SH_CB == 4,
              "chunk word offsets");
static_assert(sh_code_reg(1) == 5 && sh_code_reg(2) == 9 && sh_code_reg(3) == 14 && sh_code_reg(4) == 18,
              "code dword slots");
static_assert(2u * 17u * 4u == SH_CB * SF37_Q8_0_BYTES, "the two halves cover the chunk exactly");

__device__ __forceinline__ void sh_load(sh_half &h, const uint8_t *wrow, uint32_t c, uint32_t kh) {
    const uint32_t *q = (const uint32_t *)(wrow + (uint64_t)c * (SH_CB * SF37_Q8_0_BYTES)) + 17u * kh;
#pragma unroll
    for (uint32_t i = 0; i < 17u; i++) h.w[i] = q[i];
}

// The chunk's words in the MFMA layout: half kh needs, per block, the code
// dwords sh_code_dw(jj) + 4 kh .. (+4 or +5) and the scale dwords 0, 8, 17,
// 25.  permlane32_swap(A, B) gives [A of lanes 0-31, B of lanes 0-31] and
// [A of lanes 32-63, B of lanes 32-63]: with A = dword i and B = dword
// 4 + i of each half, the first is block 0's dword i of both halves (dword i
// for kh = 0, dword 4 + i for kh = 1), the second block 2's (17 + i, 21 + i);
// blocks 1 and 3 likewise from dwords 9 + i and 13 + i; a swap of a dword
// with itself hands both halves the scale dwords 0 and 17 (8 and 25).
__device__ __forceinline__ void sh_swap(sh_raw &r, const sh_half &h) {
#pragma unroll
    for (uint32_t i = 0; i < 5u; i++) {
        const auto v = __builtin_amdgcn_permlane32_swap(h.w[i], h.w[4u + i], false, false);
        r.c[sh_code_reg(0) + i] = v[0];
        r.c[sh_code_reg(2) + i] = v[1];
    }
#pragma unroll
    for (uint32_t i = 0; i < 4u; i++) {
        const auto v = __builtin_amdgcn_permlane32_swap(h.w[9u + i], h.w[13u + i], false, false);
        r.c[sh_code_reg(1) + i] = v[0];
        r.c[sh_code_reg(3) + i] = v[1];
    }
    const auto s0 = __builtin_amdgcn_permlane32_swap(h.w[0], h.w[0], false, false);
    const auto s1 = __builtin_amdgcn_permlane32_swap(h.w[8], h.w[8], false, false);
    r.s[0] = s0[0];
    r.s[2] = s0[1];
    r.s[1] = s1[0];
    r.s[3] = s1[1];
}

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

// One K chunk (SH_CB Q8_0 blocks) for TBW token blocks from token block tb0.
template <int TBW>
__device__ __forceinline__ void sh_chunk(const sh_raw &r, const uint8_t *act_lds, const float *xs_lds,
                                         uint32_t kh, uint32_t col, uint32_t tb0, float (*acc)[16]) {
    const uint8_t *a_row = act_lds + (32u * tb0 + col) * SH_RS;   // token row col of token block tb0
    const uint32_t sw = col & 7u;                      // the row's slot swizzle (32 i + col has the same)
    const float *x_lane = xs_lds + 32u * tb0 + 4u * kh;
    const i32x16 magic = (i32x16)SH_MAGIC_BITS;
#pragma unroll
    for (uint32_t jj = 0; jj < SH_CB; jj++) {
        const uint32_t o = sh_code_reg(jj);
        i32x4 b;
#pragma unroll
        for (int i = 0; i < 4; i++)
            b[i] = (int)((jj & 1u) ? r.c[o + i] : align_bytes(r.c[o + i + 1], r.c[o + i], 2u));
        const float ws = sf37_f16((jj & 1u) ? r.s[jj] >> 16 : r.s[jj]);
        const float nws = -SH_MAGIC * ws;
        const uint32_t slot = ((2u * jj + kh) ^ sw) * 16u;
        // the MFMAs of every token block first, so the epilogue of one block
        // runs while the matrix cores still work on the next
        i32x16 D[TBW];
#pragma unroll
        for (uint32_t i = 0; i < TBW; i++) {
            const i32x4 a = *(const i32x4 *)(a_row + i * 32u * SH_RS + slot);
            D[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, magic, 0, 0, 0);
        }
#pragma unroll
        for (uint32_t i = 0; i < TBW; i++) {
            // the whole result reinterpreted at once (a bit_cast of one
            // vector element would name the vector's storage, i.e. element 0)
            const f16v F = __builtin_bit_cast(f16v, D[i]);
#pragma unroll
            for (int jq = 0; jq < 4; jq++) {
                const float4 xv = *(const float4 *)(x_lane + jj * SH_T + 32u * i + 8u * jq);
                const float xa[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float p = __builtin_fmaf(F[4 * jq + q], ws, nws);
                    const float t = p * xa[q];
                    acc[i][4 * jq + q] = acc[i][4 * jq + q] + t;
                }
            }
        }
    }
}

// The same chunk with its LDS reads (activation operands and scales) all
// issued first and its MFMAs next, then the epilogues in block order (same
// arithmetic, same order per output).  For grids of at most two workgroups
// per CU, where about one wave per SIMD leaves the LDS and MFMA latencies
// unhidden: they are then paid once per chunk instead of once per read, at
// ~225 VGPRs.
template <int TBW>
__device__ __forceinline__ void sh_chunk_batched(const sh_raw &r, const uint8_t *act_lds, const float *xs_lds,
                                                 uint32_t kh, uint32_t col, uint32_t tb0, float (*acc)[16]) {
    const uint8_t *a_row = act_lds + (32u * tb0 + col) * SH_RS;
    const uint32_t sw = col & 7u;
    const float *x_lane = xs_lds + 32u * tb0 + 4u * kh;
    const i32x16 magic = (i32x16)SH_MAGIC_BITS;
    i32x4 a[SH_CB][TBW];
    float4 xv[SH_CB][TBW][4];
#pragma unroll
    for (uint32_t jj = 0; jj < SH_CB; jj++) {
        const uint32_t slot = ((2u * jj + kh) ^ sw) * 16u;
#pragma unroll
        for (uint32_t i = 0; i < TBW; i++) {
            a[jj][i] = *(const i32x4 *)(a_row + i * 32u * SH_RS + slot);
#pragma unroll
            for (int jq = 0; jq < 4; jq++) xv[jj][i][jq] = *(const float4 *)(x_lane + jj * SH_T + 32u * i + 8u * jq);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    i32x16 D[SH_CB][TBW];
    float ws[SH_CB], nws[SH_CB];
#pragma unroll
    for (uint32_t jj = 0; jj < SH_CB; jj++) {
        const uint32_t o = sh_code_reg(jj);
        i32x4 b;
#pragma unroll
        for (int i = 0; i < 4; i++)
            b[i] = (int)((jj & 1u) ? r.c[o + i] : align_bytes(r.c[o + i + 1], r.c[o + i], 2u));
        ws[jj] = sf37_f16((jj & 1u) ? r.s[jj] >> 16 : r.s[jj]);
        nws[jj] = -SH_MAGIC * ws[jj];
#pragma unroll
        for (uint32_t i = 0; i < TBW; i++) D[jj][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[jj][i], b, magic, 0, 0, 0);
    }
#pragma unroll
    for (uint32_t jj = 0; jj < SH_CB; jj++) {
#pragma unroll
        for (uint32_t i = 0; i < TBW; i++) {
            const f16v F = __builtin_bit_cast(f16v, D[jj][i]);
#pragma unroll
            for (int jq = 0; jq < 4; jq++) {
                const float xa[4] = {xv[jj][i][jq].x, xv[jj][i][jq].y, xv[jj][i][jq].z, xv[jj][i][jq].w};
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float p = __builtin_fmaf(F[4 * jq + q], ws[jj], nws[jj]);
                    const float t = p * xa[q];
                    acc[i][4 * jq + q] = acc[i][4 * jq + q] + t;
                }
            }
        }
    }
}

// GU: gate/up, 16 gate + 16 up rows per wave, epilogue mid = (g*sig(g))*u
// (shared clamp).  Otherwise down: 32 output rows per wave, out written
// directly.  TBW = 2: a wave takes both 32-token blocks of the tile, the
// workgroup 128 weight columns; TBW = 1 (batches whose TBW = 2 grid would
// leave CUs idle): waves 2 c and 2 c + 1 take token block 0 and 1 of the
// same 32 columns, the workgroup 64 columns.  BAT (TBW = 1 only): the chunk
// body with its reads batched (sh_chunk_batched).
template <bool GU, int TBW, bool BAT = false>
__global__ void __launch_bounds__(256, 2) sh_gemm_kernel(sh_params p) {
    static_assert(!BAT || TBW == 1, "the batched chunk body is the narrow form's");
    __shared__ __align__(16) uint8_t s_act[2][SH_BUF];
    __shared__ __align__(16) float s_xs[2][SH_CB * SH_T];
    __shared__ uint64_t s_tab[GU ? 32 : 1];    // the exp table of the SwiGLU epilogue
    static_assert(TBW == 1 || TBW == 2, "token blocks per wave");
    if (GU) sf37_stage_exp_tab(s_tab);          // read after the chunk loop's barriers
    const uint32_t tt = blockIdx.x % p.n_tt, ct = blockIdx.x / p.n_tt;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, kh = lane >> 5, col = lane & 31u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t tb0 = TBW == 2 ? 0u : (wave & 1u), cg = TBW == 2 ? wave : wave >> 1;
    constexpr uint32_t COLS = 64u * TBW;               // weight columns per workgroup
    const uint32_t t0 = tt * SH_T;
    const uint32_t nb = p.nb, nchunk = nb / SH_CB;
    // this lane's weight row
    const uint32_t wcol = GU ? ct * (COLS / 2u) + 16u * cg + (col & 15u) : ct * COLS + 32u * cg + col;
    const bool second = GU && col >= 16u;
    const uint8_t *wrow = (second ? p.w1 : p.w0) + (uint64_t)wcol * nb * SF37_Q8_0_BYTES;
    // DMA: load L = 2 wave + k fills rows 8 L .. 8 L + 7; lane l writes row
    // 8 L + l / 8, slot l % 8, which holds piece (l % 8) ^ (l / 8) of it
    uint32_t voff[2];
#pragma unroll
    for (uint32_t k = 0; k < 2u; k++) {
        const uint32_t r = 8u * (2u * wave + k) + (lane >> 3);
        const uint32_t tr = t0 + r < p.n_tok ? t0 + r : p.n_tok - 1u;
        voff[k] = tr * nb * 32u + 16u * ((lane & 7u) ^ (lane >> 3));
    }
    const uint32_t tl = t0 + lane;
    const uint32_t tok_dma = tl < p.n_tok ? tl : p.n_tok - 1u;
    const uint32_t act_l = lds_addr(&s_act[0][0]), xs_l = lds_addr(&s_xs[0][0]);
    auto issue = [&](uint32_t c) {
        const uint32_t bf = c & 1u;
#pragma unroll
        for (uint32_t k = 0; k < 2u; k++)
            lds_dma16(act_l + bf * SH_BUF + (2u * wave + k) * DMA16_SPAN, voff[k],
                      (const uint8_t *)p.act + (uint64_t)c * (SH_CB * 32u));
        lds_dma4(xs_l + bf * (SH_CB * SH_T * 4u) + wave * SH_T * 4u, tok_dma * nb * 4u,
                 (const uint8_t *)p.xs + ((uint64_t)c * SH_CB + wave) * 4u);
    };
    float acc[TBW][16];
#pragma unroll
    for (uint32_t i = 0; i < (uint32_t)TBW; i++)
#pragma unroll
        for (int r2 = 0; r2 < 16; r2++) acc[i][r2] = 0.0f;
    sh_half ha, hb;
    issue(0);
    sh_load(ha, wrow, 0, kh);
    const uint32_t last = nchunk - 1u;
    for (uint32_t c = 0; c < nchunk; c += 2u) {
        const uint32_t c1 = c + 1u < nchunk ? c + 1u : last, c2 = c + 2u < nchunk ? c + 2u : last;
        wait_vm0();
        sh_ready(ha);
        __syncthreads();
        issue(c1);
        {
            sh_raw r;
            sh_swap(r, ha);
            sh_load(hb, wrow, c1, kh);
            if constexpr (BAT) sh_chunk_batched<TBW>(r, s_act[c & 1u], s_xs[c & 1u], kh, col, tb0, acc);
            else sh_chunk<TBW>(r, s_act[c & 1u], s_xs[c & 1u], kh, col, tb0, acc);
        }
        if (c + 1u < nchunk) {
            wait_vm0();
            sh_ready(hb);
            __syncthreads();
            issue(c2);
            sh_raw r;
            sh_swap(r, hb);
            sh_load(ha, wrow, c2, kh);
            if constexpr (BAT) sh_chunk_batched<TBW>(r, s_act[(c + 1u) & 1u], s_xs[(c + 1u) & 1u], kh, col, tb0, acc);
            else sh_chunk<TBW>(r, s_act[(c + 1u) & 1u], s_xs[(c + 1u) & 1u], kh, col, tb0, acc);
        }
    }
    wait_vm0();
#pragma unroll
    for (uint32_t i = 0; i < (uint32_t)TBW; i++) {
        if constexpr (GU) {
            // lanes col and col ^ 16 hold the gate and up rows of one mid row:
            // the gate lane forms the SwiGLU of tokens r2 = k, the up lane of
            // r2 = k + 8
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float va = acc[i][k], vb = acc[i][k + 8];
                const float oa = __shfl_xor(va, 16, 64), ob = __shfl_xor(vb, 16, 64);
                const bool up_lane = col >= 16u;
                const uint32_t r2 = up_lane ? (uint32_t)k + 8u : (uint32_t)k;
                const float g = up_lane ? ob : va, u = up_lane ? vb : oa;
                const uint32_t t = t0 + 32u * (tb0 + i) + 8u * (r2 >> 2) + 4u * kh + (r2 & 3u);
                if (t < p.n_tok) p.out0[(uint64_t)t * p.rows + wcol] = sf37_swiglu_mid_t(g, u, 1.0f, p.clamp, s_tab);
            }
        } else {
#pragma unroll
            for (int r2 = 0; r2 < 16; r2++) {
                const uint32_t t = t0 + 32u * (tb0 + i) + 8u * (r2 >> 2) + 4u * kh + (r2 & 3);
                if (t < p.n_tok) p.out0[(uint64_t)t * p.rows + wcol] = acc[i][r2];
            }
        }
    }
}

uint32_t pf_grid(uint32_t max_tiles, uint32_t n_rt) { return 8u * ((max_tiles + 7u) / 8u) * n_rt; }

}  // namespace

extern "C" uint32_t sf37k_pf_max_tiles(uint32_t n_pairs, uint32_t max_groups) {
    return (n_pairs + PF_T - 1u) / PF_T + max_groups;
}

extern "C" int sf37k_pf_supported(uint32_t in_dim, uint32_t mid_dim, uint32_t out_dim) {
    return in_dim % SF37_QK == 0 && mid_dim % SF37_QK == 0 && mid_dim % PF_GU_R == 0 &&
           out_dim % PF_DN_R == 0 && in_dim > 0 && mid_dim > 0;   // 32 weight columns per wave
}

extern "C" int sf37k_pf_act(int q3, void *codes_v, float *tab, const float *x, uint32_t dim,
                            uint32_t n_rows, sf37_stream_t s) {
    _Float16 *codes = (_Float16 *)codes_v;
    const uint32_t nblk = dim / SF37_QK;
    const uint64_t units = (uint64_t)nblk * n_rows;
    if (units == 0) return 0;
    if (units > 0xffffffffu) return (int)hipErrorInvalidValue;
    // four units per workgroup pass; at most 2048 workgroups, each wave then
    // walks several units
    const uint64_t wgs = (units + 3u) / 4u;
    const dim3 grid((unsigned)(wgs < 2048u ? wgs : 2048u));
    if (q3)
        hipLaunchKernelGGL(pf_act_kernel<true>, grid, dim3(256), 0, (hipStream_t)s, codes, tab, x, nblk, n_rows);
    else
        hipLaunchKernelGGL(pf_act_kernel<false>, grid, dim3(256), 0, (hipStream_t)s, codes, tab, x, nblk, n_rows);
    return (int)hipGetLastError();
}

extern "C" uint32_t sf37k_pf_tab_stride(uint32_t n_pairs) { return (n_pairs + PF_T + 63u) & ~63u; }

extern "C" int sf37k_pf_tab_sort(float *tabs, const float *tab, const uint32_t *sorted_pairs, uint32_t n_pairs,
                                 uint32_t dim, uint32_t div, sf37_stream_t s) {
    const uint32_t nblk = dim / SF37_QK;
    if (n_pairs == 0) return 0;
    hipLaunchKernelGGL(pf_tab_sort_kernel, dim3((n_pairs + 255u) / 256u, nblk), dim3(256), 0, (hipStream_t)s, tabs,
                       tab, sorted_pairs, n_pairs, nblk, div, sf37k_pf_tab_stride(n_pairs));
    return (int)hipGetLastError();
}

extern "C" int sf37k_pf_tiles(uint32_t *tiles, const uint32_t *group_info, uint32_t max_groups,
                              sf37_stream_t s) {
    hipLaunchKernelGGL(pf_tiles_kernel, dim3(1), dim3(1024), 0, (hipStream_t)s, tiles, group_info, max_groups);
    return (int)hipGetLastError();
}

extern "C" int sf37k_pf_gate_up(float *mid, float *gate_out, float *up_out, const uint8_t *gate_w,
                                const uint8_t *up_w, const void *act, const float *tab,
                                const uint32_t *tiles, const uint32_t *sorted_pairs, const float *weights,
                                uint32_t max_tiles, uint32_t tab_stride, uint32_t topk, uint32_t in_dim,
                                uint32_t mid_dim, float clamp, sf37_stream_t s) {
    pf_params p = {};
    p.mid = mid;
    p.gate_out = gate_out;
    p.up_out = up_out;
    p.w0 = gate_w;
    p.w1 = up_w;
    p.act = (const _Float16 *)act;
    p.tab = tab;
    p.tiles = tiles;
    p.sorted = sorted_pairs;
    p.weights = weights;
    p.topk = topk;
    p.nblk = in_dim / SF37_QK;
    p.out_rows = mid_dim;
    p.n_rt = mid_dim / PF_GU_R;
    p.tab_stride = tab_stride;
    p.clamp = clamp;
    hipLaunchKernelGGL(pf_expert_kernel<true>, dim3(pf_grid(max_tiles, p.n_rt)), dim3(pf_cfg<true>::NW * 64), 0, (hipStream_t)s, p);
    return (int)hipGetLastError();
}

extern "C" int sf37k_pf_down(float *down_pair, const uint8_t *down_w, const void *act, const float *tab,
                             const uint32_t *tiles, const uint32_t *sorted_pairs, uint32_t max_tiles,
                             uint32_t tab_stride, uint32_t mid_dim, uint32_t out_dim, sf37_stream_t s) {
    pf_params p = {};
    p.down_pair = down_pair;
    p.w0 = down_w;
    p.act = (const _Float16 *)act;
    p.tab = tab;
    p.tiles = tiles;
    p.sorted = sorted_pairs;
    p.nblk = mid_dim / SF37_QK;
    p.out_rows = out_dim;
    p.n_rt = out_dim / PF_DN_R;
    p.tab_stride = tab_stride;
    hipLaunchKernelGGL(pf_expert_kernel<false>, dim3(pf_grid(max_tiles, p.n_rt)), dim3(pf_cfg<false>::NW * 64), 0, (hipStream_t)s, p);
    return (int)hipGetLastError();
}

// The 64-column shared GEMM when the 128-column grid (n_ct x n_tt
// workgroups) is under two workgroups per CU (measured crossover: at 2048
// tokens the 128-column gate/up grid of 640 workgroups takes 128 us, the
// 64-column one 157 us; at 512 tokens 64 columns win, 73 against 75 us).
static uint32_t sh_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    return (uint32_t)cus;
}
static bool sh_narrow(uint32_t n_ct, uint32_t n_tt) { return (uint64_t)n_ct * n_tt < 2ull * sh_cus(); }
// The narrow form's batched chunk body when its grid (n_ct x n_tt, 64
// columns) is one round at two workgroups per CU (measured, gate/up + down:
// 256 tokens 57 + 21 -> 46 + 16 us, 512 tokens 73 + 27 -> 70 + 24 us; at
// 1024 tokens, 1.25 rounds, 97 -> 100 us, so that grid keeps the other body).
static bool sh_batched(uint32_t n_ct, uint32_t n_tt) { return (uint64_t)n_ct * n_tt <= 2ull * sh_cus(); }

extern "C" int sf37k_sh_supported(uint32_t in_dim, uint32_t mid_dim, uint32_t out_dim) {
    return in_dim % (32u * SH_CB * 2u) == 0 && mid_dim % (32u * SH_CB * 2u) == 0 && mid_dim % 64u == 0 &&
           out_dim % 128u == 0 && in_dim > 0 && mid_dim > 0;
}

extern "C" int sf37k_sh_act(void *a8, float *xs, const float *x, uint32_t dim, uint32_t n_tok, sf37_stream_t s) {
    const uint64_t n = (uint64_t)(dim / 32u) * n_tok;
    if (n == 0) return 0;
    hipLaunchKernelGGL(sh_act_kernel, dim3((unsigned)((n + 31u) / 32u)), dim3(256), 0, (hipStream_t)s,
                       (int8_t *)a8, xs, x, dim / 32u, (uint64_t)n_tok);
    return (int)hipGetLastError();
}

extern "C" int sf37k_sh_gate_up(float *mid, const uint8_t *gate_w, const uint8_t *up_w, const void *a8,
                                const float *xs, uint32_t n_tok, uint32_t in_dim, uint32_t mid_dim, float clamp,
                                sf37_stream_t s) {
    sh_params p = {};
    p.out0 = mid;
    p.w0 = gate_w;
    p.w1 = up_w;
    p.act = (const int8_t *)a8;
    p.xs = xs;
    p.n_tok = n_tok;
    p.nb = in_dim / 32u;
    p.rows = mid_dim;
    p.n_tt = (n_tok + SH_T - 1u) / SH_T;
    p.clamp = clamp;
    if (sh_narrow(mid_dim / 64u, p.n_tt)) {
        p.n_ct = mid_dim / 32u;
        if (sh_batched(p.n_ct, p.n_tt))
            hipLaunchKernelGGL((sh_gemm_kernel<true, 1, true>), dim3(p.n_ct * p.n_tt), dim3(256), 0, (hipStream_t)s, p);
        else
            hipLaunchKernelGGL((sh_gemm_kernel<true, 1>), dim3(p.n_ct * p.n_tt), dim3(256), 0, (hipStream_t)s, p);
    } else {
        p.n_ct = mid_dim / 64u;
        hipLaunchKernelGGL((sh_gemm_kernel<true, 2>), dim3(p.n_ct * p.n_tt), dim3(256), 0, (hipStream_t)s, p);
    }
    return (int)hipGetLastError();
}

extern "C" int sf37k_sh_down(float *out, const uint8_t *down_w, const void *a8, const float *xs, uint32_t n_tok,
                             uint32_t mid_dim, uint32_t out_dim, sf37_stream_t s) {
    sh_params p = {};
    p.out0 = out;
    p.w0 = down_w;
    p.act = (const int8_t *)a8;
    p.xs = xs;
    p.n_tok = n_tok;
    p.nb = mid_dim / 32u;
    p.rows = out_dim;
    p.n_tt = (n_tok + SH_T - 1u) / SH_T;
    if (sh_narrow(out_dim / 128u, p.n_tt)) {
        p.n_ct = out_dim / 64u;
        if (sh_batched(p.n_ct, p.n_tt))
            hipLaunchKernelGGL((sh_gemm_kernel<false, 1, true>), dim3(p.n_ct * p.n_tt), dim3(256), 0, (hipStream_t)s, p);
        else
            hipLaunchKernelGGL((sh_gemm_kernel<false, 1>), dim3(p.n_ct * p.n_tt), dim3(256), 0, (hipStream_t)s, p);
    } else {
        p.n_ct = out_dim / 128u;
        hipLaunchKernelGGL((sh_gemm_kernel<false, 2>), dim3(p.n_ct * p.n_tt), dim3(256), 0, (hipStream_t)s, p);
    }
    return (int)hipGetLastError();
}
