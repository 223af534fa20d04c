// k_attn.hip — the attention half of the LLaDA2 layer on gfx950
// (src/diffuse-moe-graph.cpp:116-178), between the fused QKV projection and
// the output projection.
//
// k_qk_rope: per (token, head) one wavefront: the head's slice of the fused
//   QKV row (Q heads, then K heads, then V heads, :132-134), the QK RMSNorm
//   over head_dim times q_norm / k_norm (:141-146; binary64 sum of the f32
//   squares, as ggml_rms_norm), the partial NEOX RoPE of the first rotary_dim
//   dims at position t (:154-155): pair ic = (x[ic], x[ic + rd/2]) rotated by
//   theta = t * theta_scale^ic, the angle formed by repeated f32
//   multiplication as ggml's rope cache does (theta_scale = powf(base,
//   -2/rd), computed on the host); V heads are copied.  Output head-major:
//   Q [n_head][N][hd], K and V [n_head_kv][N][hd].
//
// k_attn: flash attention with the block-causal mask of :19-55 (query i sees
//   key j iff j / B <= i / B; every key when B <= 0), scale 1/sqrt(hd), GQA
//   query head h on kv head h / (n_head / n_head_kv) (:158-167).  One
//   workgroup per (head, 64 or 128 queries), the last query blocks (the most
//   keys) dispatched first, four or eight wavefronts of 16 queries each;
//   64-key tiles of K and V staged in LDS; S = Q K^T and O += P V on
//   v_mfma_f32_16x16x32_f16 with every f32 operand split into f16 hi + lo
//   halves (hi lo' + lo hi' + hi hi', f32 accumulation: ~2^-22 relative per
//   product, the fp32 result to within its own rounding; |values| below
//   65504, the f16 range), online softmax per query row in registers.  Keys
//   past the last block a query tile can see are not visited.
#include <type_traits>

#include "dmoe_internal.h"

#pragma clang fp contract(off)

namespace dmoe {

typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int QR_THREADS = 256;

__global__ __launch_bounds__(QR_THREADS) void k_qk_rope(const float *__restrict__ qkv, int ks, size_t kstride,
                                                        const float *__restrict__ qn,
                                                        const float *__restrict__ kn, AttnDims a,
                                                        float *__restrict__ Qh, float *__restrict__ Kh,
                                                        float *__restrict__ Vh)
{
    __shared__ float s_x[QR_THREADS / 64][256];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int heads = a.nh + 2 * a.nkv;
    const int item = blockIdx.x * (QR_THREADS / 64) + w;
    if (item >= a.n * heads) return;
    const int t = item / heads, hh = item % heads;
    const int HD = a.hd, QKV = (a.nh + 2 * a.nkv) * HD;
    const float *src = qkv + (size_t)t * QKV + (size_t)hh * HD;
    float *x = s_x[w];
    // the fused projection's row: the sum of its ks reduction slices, in order
    for (int d = lane; d < HD; d += 64) {
        float v = src[d];
        for (int k = 1; k < ks; k++) v = v + src[(size_t)k * kstride + d];
        x[d] = v;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (hh < a.nh + a.nkv) {
        if (a.qk_norm) {
            double acc = 0.0;
            for (int d = lane; d < HD; d += 64) acc += (double)(x[d] * x[d]);
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
            const float mean = (float)(acc / (double)HD);
            const float scale = 1.0f / sqrtf(mean + a.eps);
            const float *nw = hh < a.nh ? qn : kn;
            for (int d = lane; d < HD; d += 64) x[d] = (x[d] * scale) * nw[d];
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        }
        const int half = a.rd / 2;
        if (lane < half) {
            float theta = (float)t;
            for (int i = 0; i < lane; i++) theta *= a.theta_scale;
            const float c = cosf(theta), sn = sinf(theta);
            const float x0 = x[lane], x1 = x[lane + half];
            x[lane] = x0 * c - x1 * sn;
            x[lane + half] = x0 * sn + x1 * c;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }
    float *dst;
    if (hh < a.nh)
        dst = Qh + ((size_t)hh * a.n + t) * HD;
    else if (hh < a.nh + a.nkv)
        dst = Kh + ((size_t)(hh - a.nh) * a.n + t) * HD;
    else
        dst = Vh + ((size_t)(hh - a.nh - a.nkv) * a.n + t) * HD;
    for (int d = lane; d < HD; d += 64) dst[d] = x[d];
}

hipError_t launch_qk_rope(const float *qkv, int ks, size_t kstride, const float *qn, const float *kn,
                          const AttnDims &a, float *Qh, float *Kh, float *Vh, hipStream_t s)
{
    if (a.hd <= 0 || a.hd > 256 || a.rd > a.hd || a.rd % 2 || a.rd / 2 > 64 || ks < 1) return hipErrorInvalidValue;
    const int items = a.n * (a.nh + 2 * a.nkv);
    hipLaunchKernelGGL(k_qk_rope, dim3((items + 3) / 4), dim3(QR_THREADS), 0, s, qkv, ks, kstride, qn, kn, a, Qh,
                       Kh, Vh);
    return hipGetLastError();
}

constexpr int AT_K = 64;              // keys per tile
constexpr int AT_KB = AT_K / 16;      // 16-key blocks of a tile
constexpr int AT_LVT = AT_K + 16;     // f16 row stride of the transposed V tile
constexpr int AT_LP = AT_K + 8;       // f16 row stride of P

typedef _Float16 at_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 at_h4 __attribute__((ext_vector_type(4)));

// x = hi + lo with hi = f16(x) and lo = f16(x - hi) (x - hi is exact in f32):
// 22 significant bits, and hi lo' + hi' lo + hi hi' is x x' to ~2^-22
// relative (the products are exact in f32)
__device__ __forceinline__ void at_split(float x, _Float16 &hi, _Float16 &lo)
{
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// The partner of each lane in a 16-lane row by DPP (no LDS round trip):
// quad_perm [1,0,3,2] and [2,3,0,1] (lane ^ 1, lane ^ 2), then the half-row
// and row mirrors, which pair quad q with quad q ^ 1 and half h with half
// h ^ 1 as lane ^ 4 and lane ^ 8 do: after the four steps of
// v = op(v, partner) every lane holds the same tree over its row as the
// __shfl_xor butterfly over 1, 2, 4, 8 (op commutative), so the same bits.
template <int CTRL>
__device__ __forceinline__ float at_dpp(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float at_row_max(float v)
{
    v = fmaxf(v, at_dpp<0xb1>(v));
    v = fmaxf(v, at_dpp<0x4e>(v));
    v = fmaxf(v, at_dpp<0x141>(v));
    return fmaxf(v, at_dpp<0x140>(v));
}

__device__ __forceinline__ float at_row_sum(float v)
{
    v = v + at_dpp<0xb1>(v);
    v = v + at_dpp<0x4e>(v);
    v = v + at_dpp<0x141>(v);
    return v + at_dpp<0x140>(v);
}

template <int HD, int QW>
__global__ __launch_bounds__(QW * 64) void k_attn(const float *__restrict__ Qh, const float *__restrict__ Kh,
                                              const float *__restrict__ Vh, AttnDims a, float *__restrict__ out)
{
    constexpr int AT_Q = 16 * QW;     // queries per workgroup (16 per wavefront)
    constexpr int AT_T = 64 * QW;     // threads per workgroup
    // f16 hi / lo planes in LDS, rows padded so that the 16-byte operand
    // reads of a wavefront's 16 rows do not conflict: a row stride of 8 dwords
    // mod 32 (measured: 4, 12, 16 and 20 conflict) for K [key][d] (HD + 16
    // halves) and V transposed [d][key] (AT_K + 16); P [query][key] keeps
    // AT_K + 8, where its 2-byte writes by rows 4 g + i do not conflict
    // either (with AT_K + 16 they do)
    constexpr int LK = HD + 16;
    __shared__ __align__(16) _Float16 sK[2][AT_K * LK];
    __shared__ __align__(16) _Float16 sV[2][HD * AT_LVT];
    __shared__ __align__(16) _Float16 sP[AT_Q / 16][2][16 * AT_LP];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    // the grid's x is the head and y the query block, last block first: the
    // dispatch order then starts the workgroups with the most key tiles
    // (a block-causal tile row grows with its query block) and the short ones
    // fill in behind them
    const int N = a.n, h = blockIdx.x, kvh = h / (a.nh / a.nkv);
    const int q_wg = (gridDim.y - 1 - blockIdx.y) * AT_Q;
    const float *Q = Qh + (size_t)h * N * HD, *K = Kh + (size_t)kvh * N * HD, *V = Vh + (size_t)kvh * N * HD;
    // keys the workgroup's last query can see
    const int q_last = min(N, q_wg + AT_Q) - 1;
    const int k_end = a.block > 0 ? min(N, (q_last / a.block + 1) * a.block) : N;
    // scores in the base-2 domain: s' = s scale log2(e), p = 2^(s' - m') (the
    // hardware exp2; the same probabilities as exp(s scale - m) to ~1e-7)
    const float scale = a.scale * 1.44269504088896341f;
    const int q0 = q_wg + 16 * w;                      // this wavefront's first query
    // this wavefront's Q operands in registers: row q0 + r16 (zero past N),
    // dims 32 c + 8 g .. + 7 of chunk c, as hi / lo halves
    at_h8 qa[HD / 32][2];
    {
        const bool in = q0 + r16 < N;
        const float *qr = Q + (size_t)(q0 + r16) * HD + 8 * g;
#pragma unroll
        for (int c = 0; c < HD / 32; c++) {
            const float4 x0 = in ? *reinterpret_cast<const float4 *>(qr + 32 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
            const float4 x1 = in ? *reinterpret_cast<const float4 *>(qr + 32 * c + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
            const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                _Float16 hi, lo;
                at_split(xs[e], hi, lo);
                qa[c][0][e] = hi;
                qa[c][1][e] = lo;
            }
        }
    }
    float m[4], l[4];
    f4v o[HD / 16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        m[i] = -__builtin_inff();
        l[i] = 0.0f;
    }
#pragma unroll
    for (int b = 0; b < HD / 16; b++) o[b] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
    // the mask of query row i as a key limit: k / B <= q / B exactly when
    // k < (q / B + 1) B, so a key is visible iff k < kvis[i] (no division per
    // score)
    int kvis[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int q = q0 + 4 * g + i;
        kvis[i] = a.block > 0 ? min(N, (q / a.block + 1) * a.block) : N;
    }
    // keys the wavefront's last query can see
    const int qw_last = min(N, q0 + 16) - 1;
    const int kw_end = a.block > 0 ? min(N, (qw_last / a.block + 1) * a.block) : N;
    // K and V tiles: the next tile's loads go to registers while the current
    // one is in use, and to LDS (split, V transposed) once every wavefront is
    // done with it.  K piece j of a thread: row i / (HD / 4), dims 4 (i %
    // (HD / 4)) .. + 3 (i = tid + AT_T j); V piece pair j: rows 2 p and 2 p + 1
    // (p = i % (AT_K / 2)), the same four dims 4 (i / (AT_K / 2)) .. + 3, so
    // that the transposed stores write two keys per 32-bit word
    constexpr int KPT = AT_K * HD / 4 / AT_T;          // pieces per thread and tile
    static_assert(KPT % 2 == 0 && KPT * AT_T * 4 == AT_K * HD, "whole piece pairs per thread");
    float4 kr[KPT], vr[KPT];
    auto load_kv = [&](int row0) {
#pragma unroll
        for (int j = 0; j < KPT; j++) {
            const int i = tid + AT_T * j, r = i / (HD / 4), c = i % (HD / 4);
            kr[j] = row0 + r < N ? *reinterpret_cast<const float4 *>(K + (size_t)(row0 + r) * HD + 4 * c)
                                 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int j = 0; j < KPT / 2; j++) {
            const int i = tid + AT_T * j, p = i % (AT_K / 2), c = i / (AT_K / 2);
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int r = 2 * p + u;
                vr[2 * j + u] = row0 + r < N ? *reinterpret_cast<const float4 *>(V + (size_t)(row0 + r) * HD + 4 * c)
                                             : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
        }
    };
    auto store_kv = [&]() {
#pragma unroll
        for (int j = 0; j < KPT; j++) {
            const int i = tid + AT_T * j, r = i / (HD / 4), c = i % (HD / 4);
            const float x[4] = {kr[j].x, kr[j].y, kr[j].z, kr[j].w};
            at_h4 hi, lo;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                _Float16 a0, a1;
                at_split(x[e], a0, a1);
                hi[e] = a0;
                lo[e] = a1;
            }
            *reinterpret_cast<at_h4 *>(&sK[0][r * LK + 4 * c]) = hi;
            *reinterpret_cast<at_h4 *>(&sK[1][r * LK + 4 * c]) = lo;
        }
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
        for (int j = 0; j < KPT / 2; j++) {
            const int i = tid + AT_T * j, p = i % (AT_K / 2), c = i / (AT_K / 2);
            const float x0[4] = {vr[2 * j].x, vr[2 * j].y, vr[2 * j].z, vr[2 * j].w};
            const float x1[4] = {vr[2 * j + 1].x, vr[2 * j + 1].y, vr[2 * j + 1].z, vr[2 * j + 1].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                _Float16 h0, l0, h1, l1;
                at_split(x0[e], h0, l0);
                at_split(x1[e], h1, l1);
                *reinterpret_cast<h2 *>(&sV[0][(4 * c + e) * AT_LVT + 2 * p]) = h2{h0, h1};
                *reinterpret_cast<h2 *>(&sV[1][(4 * c + e) * AT_LVT + 2 * p]) = h2{l0, l1};
            }
        }
    };
    if (k_end > 0) load_kv(0);
    for (int k0 = 0; k0 < k_end; k0 += AT_K) {
        // every wavefront is done with the previous tile; this one (loaded
        // during the previous tile's products) to LDS; then the next one's
        // loads, in flight during this tile's products
        __syncthreads();
        store_kv();
        __syncthreads();
        if (k0 + AT_K < k_end) load_kv(k0 + AT_K);
        // a wavefront whose queries are all past N, and key tiles, blocks and
        // chunks wholly past its last query's last visible key, have nothing
        // to add (their probabilities are 0): skipped
        if (q0 >= N || k0 >= kw_end) continue;
        const int nkb = min(AT_KB, (kw_end - k0 + 15) / 16);
        const int npc = min(AT_K / 32, (kw_end - k0 + 31) / 32);
        // S[16 q][AT_K k]: lane holds rows 4g + i of key block kb, key kb*16 + r16
        f4v sacc[AT_KB];
#pragma unroll
        for (int kb = 0; kb < AT_KB; kb++) sacc[kb] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
        auto qk = [&](auto nkb_c) {
            constexpr int NKB = decltype(nkb_c)::value;
#pragma unroll
            for (int c = 0; c < HD / 32; c++)
#pragma unroll
                for (int kb = 0; kb < NKB; kb++) {
                    const int off = (kb * 16 + r16) * LK + 32 * c + 8 * g;
                    const at_h8 kh = *reinterpret_cast<const at_h8 *>(&sK[0][off]);
                    const at_h8 kl = *reinterpret_cast<const at_h8 *>(&sK[1][off]);
                    sacc[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[c][1], kh, sacc[kb], 0, 0, 0);
                    sacc[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[c][0], kl, sacc[kb], 0, 0, 0);
                    sacc[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[c][0], kh, sacc[kb], 0, 0, 0);
                }
        };
        static_assert(AT_KB == 4, "a tile of four 16-key blocks");
        switch (nkb) {
        case 1: qk(std::integral_constant<int, 1>{}); break;
        case 2: qk(std::integral_constant<int, 2>{}); break;
        case 3: qk(std::integral_constant<int, 3>{}); break;
        default: qk(std::integral_constant<int, 4>{}); break;
        }
        // scale, mask, online softmax per query row (rows 4g + i of the wave)
        float mt[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float mx = -__builtin_inff();
#pragma unroll
            for (int kb = 0; kb < AT_KB; kb++) {
                const int k = k0 + kb * 16 + r16;
                const bool ok = k < kvis[i];
                const float v = ok ? sacc[kb][i] * scale : -__builtin_inff();
                sacc[kb][i] = v;
                mx = fmaxf(mx, v);
            }
            mt[i] = at_row_max(mx);
        }
        float corr[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float mn = fmaxf(m[i], mt[i]);
            // a row with no visible key yet keeps m = -inf and contributes 0
            corr[i] = mn == -__builtin_inff() ? 1.0f : __builtin_amdgcn_exp2f(m[i] - mn);
            float rs = 0.0f;
#pragma unroll
            for (int kb = 0; kb < AT_KB; kb++) {
                const float p = mn == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(sacc[kb][i] - mn);
                sacc[kb][i] = p;
                rs += p;
            }
            rs = at_row_sum(rs);
            l[i] = l[i] * corr[i] + rs;
            m[i] = mn;
        }
#pragma unroll
        for (int b = 0; b < HD / 16; b++)
#pragma unroll
            for (int i = 0; i < 4; i++) o[b][i] *= corr[i];
        // P to LDS as hi / lo halves in the layout of the next product's A
        // operand (row = query, 16-byte pieces of 8 keys)
        _Float16 *ph = sP[w][0], *pl = sP[w][1];
#pragma unroll
        for (int kb = 0; kb < AT_KB; kb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                _Float16 hi, lo;
                at_split(sacc[kb][i], hi, lo);
                ph[(4 * g + i) * AT_LP + kb * 16 + r16] = hi;
                pl[(4 * g + i) * AT_LP + kb * 16 + r16] = lo;
            }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        // O[16 q][HD] += P[16 q][AT_K k] V[AT_K k][HD], 32 keys per chunk
        auto pv = [&](auto npc_c) {
            constexpr int NPC = decltype(npc_c)::value;
#pragma unroll
            for (int c = 0; c < NPC; c++) {
                const int po = r16 * AT_LP + 32 * c + 8 * g;
                const at_h8 pah = *reinterpret_cast<const at_h8 *>(ph + po);
                const at_h8 pal = *reinterpret_cast<const at_h8 *>(pl + po);
#pragma unroll
                for (int b = 0; b < HD / 16; b++) {
                    const int vo = (b * 16 + r16) * AT_LVT + 32 * c + 8 * g;
                    const at_h8 vh = *reinterpret_cast<const at_h8 *>(&sV[0][vo]);
                    const at_h8 vl = *reinterpret_cast<const at_h8 *>(&sV[1][vo]);
                    o[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pal, vh, o[b], 0, 0, 0);
                    o[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pah, vl, o[b], 0, 0, 0);
                    o[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pah, vh, o[b], 0, 0, 0);
                }
            }
        };
        static_assert(AT_K == 64, "a tile of two 32-key chunks");
        if (npc == 2)
            pv(std::integral_constant<int, 2>{});
        else
            pv(std::integral_constant<int, 1>{});
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }
    // out[t][h*HD + d] = O / l (lane: rows 4g + i, column b*16 + r16)
    const int QD = a.nh * HD;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int q = q0 + 4 * g + i;
        if (q >= N) continue;
        const float inv = l[i];
#pragma unroll
        for (int b = 0; b < HD / 16; b++) out[(size_t)q * QD + (size_t)h * HD + b * 16 + r16] = o[b][i] / inv;
    }
}

hipError_t launch_attn(const float *Qh, const float *Kh, const float *Vh, const AttnDims &a, float *out,
                       hipStream_t s)
{
    if (a.nkv <= 0 || a.nh % a.nkv || (a.waves != 0 && a.waves != 4 && a.waves != 8)) return hipErrorInvalidValue;
    // eight wavefronts (128 queries) per workgroup once that still gives two
    // workgroups per CU (each K / V tile staged once for twice the queries),
    // else four (more workgroups for the few-query grids)
    int n_cu = 0;
    const hipError_t e = device_cu_count(&n_cu);
    if (e != hipSuccess) return e;
    const bool wide = a.waves ? a.waves == 8 : (long)a.nh * ((a.n + 127) / 128) >= 2L * n_cu;
    const dim3 grid(a.nh, (a.n + (wide ? 127 : 63)) / (wide ? 128 : 64));
    switch (a.hd * (wide ? -1 : 1)) {
    case 64: hipLaunchKernelGGL((k_attn<64, 4>), grid, dim3(256), 0, s, Qh, Kh, Vh, a, out); break;
    case 128: hipLaunchKernelGGL((k_attn<128, 4>), grid, dim3(256), 0, s, Qh, Kh, Vh, a, out); break;
    case -64: hipLaunchKernelGGL((k_attn<64, 8>), grid, dim3(512), 0, s, Qh, Kh, Vh, a, out); break;
    case -128: hipLaunchKernelGGL((k_attn<128, 8>), grid, dim3(512), 0, s, Qh, Kh, Vh, a, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

} // namespace dmoe
