// k_gemm.hip — grouped F16 expert products on MFMA (gfx950), the prefill path.
//
// Computes the routed experts of src/diffuse-moe-graph.cpp:264-269 for F16
// expert weights (ggml's mul_mat_id converts the activations to F16, its
// vec_dot_type, and accumulates f16 x f16 products in f32) and the shared
// expert of :280-286 (F32 semantics: its F16 weights are exact, the f32
// activations run as two f16 passes, hi = f16(x) and lo = f16(x - hi)):
//   phase 0: h = silu(W_gate x) * (W_up x), written as the f16 activations of
//            phase 1 (routed) or as their hi / lo pair (shared)
//   phase 1: y = W_down h
//
// Work item: one expert, a block of up to 128 of its (token, slot) pairs (or
// 128 tokens of the shared expert) and a group of output rows (64 moe_ff rows
// of gate and of up, or 128 n_embd rows of down).  Items of one expert and
// row group but different pair blocks are a row-group count apart, so they run
// together and share the weight rows through the caches.  Each 32-wide k
// step stages the 128 activation rows and the 128 weight rows through
// double-buffered LDS; every wavefront computes a 64 x 64 output tile as 4 x 4
// v_mfma_f32_16x16x32_f16 (operand layout as in k_expert.hip: srcA lane l =
// activation row l%16, k = 8*(l/16)+e; srcB = weight row, same k; D lane l =
// weight row l%16, activation rows 4*(l/16)+i).
#include "dmoe_internal.h"

namespace dmoe {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int GWAVES = 4;
constexpr int GT = GWAVES * 64;      // threads per workgroup
constexpr int GROW = GK + 8;         // LDS row (f16) with padding: 80 bytes, conflict-free reads

__device__ __forceinline__ float gsilu(float g) { return g / (1.0f + __expf(-g)); }

__device__ __forceinline__ uint16_t f2h_rn(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

template <int PHASE>
__global__ __launch_bounds__(GT) void k_gemm_f16(GemmJob job)
{
    constexpr bool DOWN = PHASE == 1;
    constexpr int GN = DOWN ? GN_DN : GN_GU;         // output rows per item
    __shared__ __align__(16) uint16_t As[2][GM][GROW];
    __shared__ __align__(16) uint16_t Bs[2][128][GROW];
    __shared__ int s_arow[GM];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r16 = lane & 15;
    const int N = job.n_tokens, K = job.top_k;
    const int H = job.H, FF = job.FF, SF = job.SF;
    const int n_ec = job.wl.n_ec[0];
    const int nch = job.has_shared ? (N + GM - 1) / GM : 0;
    const int rg = (DOWN ? H : FF) / GN, rg_sh = (DOWN ? H : SF) / GN;
    const int routed_items = n_ec * rg;
    const int total = routed_items + nch * rg_sh;
    const int tok0 = 64 * (wave >> 1);               // this wave's 64 activation rows

    for (int item = blockIdx.x; item < total; item += gridDim.x) {
        const bool shared = item >= routed_items;
        const int j = shared ? item - routed_items : item;
        const int rgn = shared ? rg_sh : rg;
        const int unit = j / rgn, rb = j - unit * rgn;
        int t_first, nt, e = 0;
        if (!shared) {
            e = job.wl.ec_expert[unit];
            const int c0 = job.wl.ec_chunk[unit] * GM;
            t_first = job.offsets[e] + c0;
            nt = min(GM, job.counts[e] - c0);
        } else {
            t_first = unit * GM;
            nt = min(GM, N - t_first);
        }
        const int Kin = DOWN ? (shared ? SF : FF) : H;
        const int nsteps = Kin / GK;
        const int total_steps = (shared ? 2 : 1) * nsteps;
        // activations: rows of a [rows][Kin] f16 array (split: lo rows after the hi rows)
        const uint16_t *A = DOWN ? (shared ? job.hs16 : job.h16) : (shared ? job.xs16 : job.x16);
        const size_t lo_off = (size_t)N * Kin;           // split arrays only

        __syncthreads();                                  // previous item's LDS reads are done
        if (tid < GM) {
            const int i = min(tid, nt - 1);
            int row;
            if (shared) {
                row = t_first + i;
            } else {
                const int p = job.perm[t_first + i];
                row = DOWN ? p : p / K;
            }
            s_arow[tid] = row;
        }
        __syncthreads();

        // this thread's two 16-byte pieces of each tile: row c >> 2, column (c & 3) * 8
        const int pr0 = tid >> 2, pr1 = (tid + GT) >> 2, pc = (tid & 3) * 8;
        const uint16_t *a0 = A + (size_t)s_arow[pr0] * Kin + pc;
        const uint16_t *a1 = A + (size_t)s_arow[pr1] * Kin + pc;
        // weight row r (0..127) of this item: gate rows 0..63 and up rows 64..127
        // of the same moe_ff rows, or 128 down rows
        auto wrow = [&](int r) -> const uint8_t * {
            if (!DOWN) {
                const WTensor &w = r < 64 ? (shared ? job.sg : job.eg) : (shared ? job.su : job.eu);
                const int rr = r < 64 ? r : r - 64;
                return w.data + (size_t)e * w.nb2 + (size_t)(rb * GN + rr) * w.nb1;
            }
            const WTensor &w = shared ? job.sd : job.ed;
            return w.data + (size_t)e * w.nb2 + (size_t)(rb * GN + r) * w.nb1;
        };
        const uint8_t *b0 = wrow(pr0) + pc * 2, *b1 = wrow(pr1) + pc * 2;

        auto gload = [&](int st, uint4 (&va)[2], uint4 (&vb)[2]) {
            const int pass = st >= nsteps ? 1 : 0;
            const int k0 = (st - pass * nsteps) * GK;
            const size_t off = pass ? lo_off : 0;
            va[0] = *reinterpret_cast<const uint4 *>(a0 + off + k0);
            va[1] = *reinterpret_cast<const uint4 *>(a1 + off + k0);
            vb[0] = *reinterpret_cast<const uint4 *>(b0 + (size_t)k0 * 2);
            vb[1] = *reinterpret_cast<const uint4 *>(b1 + (size_t)k0 * 2);
        };
        auto lstore = [&](int buf, const uint4 (&va)[2], const uint4 (&vb)[2]) {
            *reinterpret_cast<uint4 *>(&As[buf][pr0][pc]) = va[0];
            *reinterpret_cast<uint4 *>(&As[buf][pr1][pc]) = va[1];
            *reinterpret_cast<uint4 *>(&Bs[buf][pr0][pc]) = vb[0];
            *reinterpret_cast<uint4 *>(&Bs[buf][pr1][pc]) = vb[1];
        };

        f4 acc[4][4];
#pragma unroll
        for (int ti = 0; ti < 4; ti++)
#pragma unroll
            for (int tw = 0; tw < 4; tw++) acc[ti][tw] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
        // weight rows of this wave's four 16-row tiles in Bs
        int brow[4];
#pragma unroll
        for (int tw = 0; tw < 4; tw++)
            brow[tw] = DOWN ? 64 * (wave & 1) + 16 * tw
                            : (tw < 2 ? 32 * (wave & 1) + 16 * tw : 64 + 32 * (wave & 1) + 16 * (tw - 2));

        {
            uint4 va[2], vb[2];
            gload(0, va, vb);
            lstore(0, va, vb);
        }
        __syncthreads();
        for (int st = 0; st < total_steps; st++) {
            const int buf = st & 1;
            uint4 va[2], vb[2];
            gload(min(st + 1, total_steps - 1), va, vb);  // clamped: every step loads
            h8 a[4], b[4];
#pragma unroll
            for (int ti = 0; ti < 4; ti++)
                a[ti] = *reinterpret_cast<const h8 *>(&As[buf][tok0 + 16 * ti + r16][8 * g]);
#pragma unroll
            for (int tw = 0; tw < 4; tw++)
                b[tw] = *reinterpret_cast<const h8 *>(&Bs[buf][brow[tw] + r16][8 * g]);
#pragma unroll
            for (int ti = 0; ti < 4; ti++)
#pragma unroll
                for (int tw = 0; tw < 4; tw++)
                    acc[ti][tw] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[ti], b[tw], acc[ti][tw], 0, 0, 0);
            if (st + 1 < total_steps) lstore(buf ^ 1, va, vb);
            __syncthreads();
        }

        // results: output row of tile tw for lane r16; activation rows 16 ti + 4 g + i
#pragma unroll
        for (int ti = 0; ti < 4; ti++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tt = tok0 + 16 * ti + 4 * g + i;
                if (tt >= nt) continue;
                if (!DOWN) {
#pragma unroll
                    for (int tj = 0; tj < 2; tj++) {
                        const int row = rb * GN + 32 * (wave & 1) + 16 * tj + r16;
                        const float hv = gsilu(acc[ti][tj][i]) * acc[ti][2 + tj][i];
                        if (!shared) {
                            const int p = job.perm[t_first + tt];
                            job.h16[(size_t)p * FF + row] = f2h_rn(hv);
                        } else {
                            const int t = t_first + tt;
                            const uint16_t hi = f2h_rn(hv);
                            job.hs16[(size_t)t * SF + row] = hi;
                            job.hs16[(size_t)N * SF + (size_t)t * SF + row] =
                                f2h_rn(hv - (float)__builtin_bit_cast(_Float16, hi));
                        }
                    }
                } else {
                    float *o = shared ? job.ys + (size_t)(t_first + tt) * H
                                      : job.ye + (size_t)job.perm[t_first + tt] * H;
#pragma unroll
                    for (int tw = 0; tw < 4; tw++) o[rb * GN + brow[tw] + r16] = acc[ti][tw][i];
                }
            }
    }
}

// x (f32 rows) -> f16 rows, or the hi / lo f16 pair (lo rows after the hi rows)
__global__ __launch_bounds__(256) void k_cvt_f16(const float *__restrict__ src, size_t n, int split,
                                                 uint16_t *__restrict__ dst)
{
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= n) return;
    const float4 v = *reinterpret_cast<const float4 *>(src + i);
    const float x[4] = {v.x, v.y, v.z, v.w};
    uint16_t hi[4], lo[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        hi[k] = f2h_rn(x[k]);
        lo[k] = f2h_rn(x[k] - (float)__builtin_bit_cast(_Float16, hi[k]));
    }
    uint2 ph, pl;
    ph.x = (uint32_t)hi[0] | ((uint32_t)hi[1] << 16);
    ph.y = (uint32_t)hi[2] | ((uint32_t)hi[3] << 16);
    *reinterpret_cast<uint2 *>(dst + i) = ph;
    if (split) {
        pl.x = (uint32_t)lo[0] | ((uint32_t)lo[1] << 16);
        pl.y = (uint32_t)lo[2] | ((uint32_t)lo[3] << 16);
        *reinterpret_cast<uint2 *>(dst + n + i) = pl;
    }
}

hipError_t launch_cvt_f16(const float *src, int rows, int K, int split, uint16_t *dst, hipStream_t s)
{
    const size_t n = (size_t)rows * K;
    if (K % 4) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_cvt_f16, dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0, s, src, n, split, dst);
    return hipGetLastError();
}

bool gemm_shapes_ok(int H, int FF, int SF, bool shared)
{
    return H % GN_DN == 0 && H % GK == 0 && FF % GN_GU == 0 && FF % GK == 0 &&
           (!shared || (SF % GN_GU == 0 && SF % GK == 0));
}

hipError_t launch_gemm_f16(int phase, const GemmJob &job, hipStream_t s)
{
    if (!gemm_shapes_ok(job.H, job.FF, job.SF, job.has_shared)) return hipErrorInvalidValue;
    if (phase == 0)
        hipLaunchKernelGGL(k_gemm_f16<0>, dim3(GEMM_BLOCKS), dim3(GT), 0, s, job);
    else
        hipLaunchKernelGGL(k_gemm_f16<1>, dim3(GEMM_BLOCKS), dim3(GT), 0, s, job);
    return hipGetLastError();
}

} // namespace dmoe
