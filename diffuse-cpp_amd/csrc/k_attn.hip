// k_attn.hip — the attention half of the LLaDA2 layer on gfx950
// (src/diffuse-moe-graph.cpp:116-178), between the fused QKV projection and
// the output projection (both run on the expert kernels' shared-down path).
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
//   workgroup per (head, 64 queries), the last query blocks (the most keys)
//   dispatched first, four wavefronts of 16 queries each;
//   64-key tiles of K and V staged in LDS; S = Q K^T and O += P V on
//   v_mfma_f32_16x16x4f32 (fp32 operands and accumulation), online softmax
//   per query row in registers.  Keys past the last block a query tile can
//   see are not visited.
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

constexpr int AT_Q = 64;              // queries per workgroup (16 per wavefront)
constexpr int AT_K = 64;              // keys per tile
constexpr int AT_KB = AT_K / 16;      // 16-key blocks of a tile

template <int HD>
__global__ __launch_bounds__(256) void k_attn(const float *__restrict__ Qh, const float *__restrict__ Kh,
                                              const float *__restrict__ Vh, AttnDims a, float *__restrict__ out)
{
    // padded LDS rows, so that the 64 lanes of an operand read hit 64
    // different banks: Q and K are read at row r16, column 4 s + g (a row
    // stride of 4 mod 64 words spreads them), V at row 4 s + g, column
    // 16 b + r16 (16 mod 64), P like Q
    constexpr int LD = HD + 4;
    constexpr int LDV = HD + 16;
    constexpr int LDP = AT_K + 4;
    __shared__ __align__(16) float sQ[AT_Q * LD];
    __shared__ __align__(16) float sK[AT_K * LD];
    __shared__ __align__(16) float sV[AT_K * LDV];
    __shared__ float sP[4][16 * LDP];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    // the grid's x is the head and y the query block, last block first: the
    // dispatch order then starts the workgroups with the most key tiles
    // (a block-causal tile row grows with its query block) and the short ones
    // fill in behind them
    const int N = a.n, h = blockIdx.x, kvh = h / (a.nh / a.nkv);
    const int q_wg = (gridDim.y - 1 - blockIdx.y) * AT_Q;
    const float *Q = Qh + (size_t)h * N * HD, *K = Kh + (size_t)kvh * N * HD, *V = Vh + (size_t)kvh * N * HD;
    // 16-byte pieces of a tile of ROWS rows of HD floats (the queries' 64,
    // a key tile's AT_K): every thread's pieces are loaded before any is
    // stored, so the loads overlap
    auto stage_tile = [&](auto rows_c, const float *src, int row0, float *dst, int ld) {
        constexpr int ROWS = decltype(rows_c)::value;
        constexpr int PPT = ROWS * HD / 4 / 256;          // pieces per thread
        static_assert(PPT * 256 * 4 == ROWS * HD, "whole pieces per thread");
        float4 v[PPT];
#pragma unroll
        for (int j = 0; j < PPT; j++) {
            const int i = tid + 256 * j, r = i / (HD / 4), c = i % (HD / 4);
            v[j] = row0 + r < N ? *reinterpret_cast<const float4 *>(src + (size_t)(row0 + r) * HD + 4 * c)
                                : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int j = 0; j < PPT; j++) {
            const int i = tid + 256 * j, r = i / (HD / 4), c = i % (HD / 4);
            *reinterpret_cast<float4 *>(dst + r * ld + 4 * c) = v[j];
        }
    };
    // queries of the workgroup (rows past N: zero)
    stage_tile(std::integral_constant<int, AT_Q>{}, Q, q_wg, sQ, LD);
    // keys the workgroup's last query can see
    const int q_last = min(N, q_wg + AT_Q) - 1;
    const int k_end = a.block > 0 ? min(N, (q_last / a.block + 1) * a.block) : N;
    // scores in the base-2 domain: s' = s scale log2(e), p = 2^(s' - m') (the
    // hardware exp2; the same probabilities as exp(s scale - m) to ~1e-7)
    const float scale = a.scale * 1.44269504088896341f;
    const int q0 = q_wg + 16 * w;                      // this wavefront's first query
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
    // K and V tiles: the next tile's loads go to registers while the current
    // one is in use, and to LDS once every wavefront is done with it
    constexpr int KPT = AT_K * HD / 4 / 256;           // pieces per thread and tile
    float4 kv[2][KPT];
    auto load_kv = [&](int row0) {
#pragma unroll
        for (int j = 0; j < KPT; j++) {
            const int i = tid + 256 * j, r = i / (HD / 4), c = i % (HD / 4);
            const bool in = row0 + r < N;
            const size_t off = (size_t)(row0 + r) * HD + 4 * c;
            kv[0][j] = in ? *reinterpret_cast<const float4 *>(K + off) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            kv[1][j] = in ? *reinterpret_cast<const float4 *>(V + off) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    auto store_kv = [&]() {
#pragma unroll
        for (int j = 0; j < KPT; j++) {
            const int i = tid + 256 * j, r = i / (HD / 4), c = i % (HD / 4);
            *reinterpret_cast<float4 *>(sK + r * LD + 4 * c) = kv[0][j];
            *reinterpret_cast<float4 *>(sV + r * LDV + 4 * c) = kv[1][j];
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
        // a wavefront whose queries are all past N, and key blocks / steps
        // wholly past the last visible key, have nothing to add (their
        // probabilities are 0): skipped
        if (q0 >= N) continue;
        const int nkb = min(AT_KB, (k_end - k0 + 15) / 16);
        const int nps = min(AT_K / 4, (k_end - k0 + 3) / 4);
        // S[16 q][AT_K k]: lane holds rows 4g + i of key block kb, key kb*16 + r16
        f4v sacc[AT_KB];
#pragma unroll
        for (int kb = 0; kb < AT_KB; kb++) sacc[kb] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
        const float *qrow = sQ + (16 * w + r16) * LD;
        auto qk = [&](auto nkb_c) {
            constexpr int NKB = decltype(nkb_c)::value;
#pragma unroll 4
            for (int s = 0; s < HD / 4; s++) {
                const float av = qrow[4 * s + g];
#pragma unroll
                for (int kb = 0; kb < NKB; kb++) {
                    const float bv = sK[(kb * 16 + r16) * LD + 4 * s + g];
                    sacc[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, sacc[kb], 0, 0, 0);
                }
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
#pragma unroll
            for (int sh = 1; sh < 16; sh <<= 1) mx = fmaxf(mx, __shfl_xor(mx, sh, 16));
            mt[i] = mx;
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
#pragma unroll
            for (int sh = 1; sh < 16; sh <<= 1) rs += __shfl_xor(rs, sh, 16);
            l[i] = l[i] * corr[i] + rs;
            m[i] = mn;
        }
#pragma unroll
        for (int b = 0; b < HD / 16; b++)
#pragma unroll
            for (int i = 0; i < 4; i++) o[b][i] *= corr[i];
        // P to LDS in the layout of the next product's A operand
        float *pw = sP[w];
#pragma unroll
        for (int kb = 0; kb < AT_KB; kb++)
#pragma unroll
            for (int i = 0; i < 4; i++) pw[(4 * g + i) * LDP + kb * 16 + r16] = sacc[kb][i];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        // O[16 q][HD] += P[16 q][AT_K k] V[AT_K k][HD]
        auto pv = [&](int ns) {
#pragma unroll 4
            for (int s = 0; s < ns; s++) {
                const float av = pw[r16 * LDP + 4 * s + g];
                const float *vrow = sV + (4 * s + g) * LDV;
#pragma unroll
                for (int b = 0; b < HD / 16; b++)
                    o[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, vrow[b * 16 + r16], o[b], 0, 0, 0);
            }
        };
        if (nps == AT_K / 4)
            pv(AT_K / 4);
        else
            pv(nps);
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
    if (a.nkv <= 0 || a.nh % a.nkv) return hipErrorInvalidValue;
    const dim3 grid(a.nh, (a.n + AT_Q - 1) / AT_Q);
    switch (a.hd) {
    case 64: hipLaunchKernelGGL(k_attn<64>, grid, dim3(256), 0, s, Qh, Kh, Vh, a, out); break;
    case 128: hipLaunchKernelGGL(k_attn<128>, grid, dim3(256), 0, s, Qh, Kh, Vh, a, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

} // namespace dmoe
