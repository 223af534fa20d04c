// k_expert_q80.hip — grouped Q8_0 expert products on int8 MFMA (gfx950).
//
// Computes the routed experts of src/diffuse-moe-graph.cpp:264-269 for Q8_0
// expert weights (ggml's mul_mat_id with Q8_0 activations, its vec_dot_type)
// and the shared expert of :280-286 (F32 semantics: the Q8_0 weights are
// exact, the f32 activations run as two int8 digit rows), as one persistent
// launch per phase:
//   phase 0: h = silu(W_gate x) * (W_up x)
//   phase 1: y = W_down h
//
// Arithmetic (ggml's vec_dot_q8_0_q8_0): per 32-value block j,
//   sum += (float)(sum_k q_w q_x) * (d_w * d_x),
// the integer dot from one v_mfma_i32_16x16x32_i8, d_w and d_x the fp16 scales
// as f32 (their product is exact in f32), blocks accumulated in order.
//
// Operand layout as in k_expert.hip (srcA lane l = activation row l%16,
// k = 8*(l/16) + byte; srcB lane l = weight row l%16, same k; D lane l = weight
// row l%16, activation rows 4*(l/16)+i).  Activations (ActI8, k_prep.hip):
// per 256 values, position 64g + 8j + b holds value 32j + 8g + b; one scale
// per 32 values.
//
// Tiled weights (k_tile_q80, at layer creation): per matrix, 16-row tiles,
// 256-value-step-major: the 16 rows x 256 values of step sb of tile t are one
// 4352-byte run at (t * nsb + sb) * 4352.  A row's 272 bytes of that step are
// seventeen 16-byte pieces, piece k of row r at (16k + r) * 16: piece 0 the
// eight fp16 scales, pieces 1 + 4g .. 4 + 4g lane group g's quants (byte 8j + b
// of the group's 64 = quant 8g + b of block j).  Same byte count as the GGUF
// blocks (8 x 34).
//
// Memory: a workgroup's eight wavefronts share one work item (16 activation
// rows).  Per step each wavefront copies its own 4352-byte tile run into a
// private 3-stage LDS ring, and six of them copy the step's activations (16
// rows x 256 int8, 16 x 8 scales) into the workgroup's 3-stage ring, with
// LDS-direct loads; one barrier per step publishes the activations.
#include "dmoe_prep.h"
#include "dmoe_q80.h"

namespace dmoe {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int Q8_WAVES = 8;                          // wavefronts per workgroup
constexpr int Q8_IT_GU = 4;                          // gate/up passes: gate, up of rows 0..127, of 128..255
constexpr int Q8_IT_DN = 2;                          // down passes: two 16-row tiles a wavefront
constexpr int Q8_GROWS_GU = Q8_WAVES * 16 * 2;       // gate/up rows of an item: one h super-block
constexpr int Q8_GROWS_DN = Q8_WAVES * 16 * Q8_IT_DN; // down rows
constexpr int Q8_STEP_ROW = 8 * Q8_0_BYTES;          // 272 bytes of a row per 256 values
constexpr int Q8_TILE = 16 * Q8_STEP_ROW;            // 4352 bytes: one tile, one step
constexpr int Q8_WPIECES = Q8_TILE / 16;             // 272
constexpr int Q8_WDMA = (Q8_WPIECES + 63) / 64;      // 5 loads per step
constexpr int Q8_STAGES = 3;
constexpr int Q8_ABYTES = 4096 + 512;                // q [16][256] + d [8][16] f32
constexpr int Q8_AD_OFF = 4096;
constexpr int Q8_BLOCKS = 1024;                      // persistent grid
static_assert(Q8_0_BYTES == 34 && Q8_STEP_ROW == 272, "Q8_0 block");

// LDS-direct loads of 16 / 4 bytes per active lane: lane l's bytes go to LDS
// address lds + 16 l (+ 4 l), lds wave-uniform.  Inline assembly so that the
// compiler does not order later LDS reads after them; completion is awaited
// with an explicit s_waitcnt on the vector-memory counter.
__device__ __forceinline__ void q8_lds_load16(const void *src, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                 : : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
}
// the same for weight runs, streamed once per forward: non-temporal hint
__device__ __forceinline__ void q8_lds_load16_nt(const void *src, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt"
                 : : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
}
__device__ __forceinline__ void q8_lds_load4(const void *src, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off"
                 : : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
}
__device__ __forceinline__ uint32_t q8_lds_addr(const void *p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// s_waitcnt with vmcnt(n) (n < 16), lgkmcnt(0), expcnt untouched
#define Q8_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(0x70 | (n))

__device__ __forceinline__ float q8_silu(float g) { return g / (1.0f + __expf(-g)); }
__device__ __forceinline__ float q8_h2f(uint32_t u) { return (float)__builtin_bit_cast(_Float16, (uint16_t)u); }

// GGUF Q8_0 rows -> tiled layout.  One thread per (row, 256-value step).
__global__ __launch_bounds__(256) void k_tile_q80(const uint8_t *__restrict__ src, size_t nb1, size_t nb2,
                                                  int rows, int nsb, int mats, uint8_t *__restrict__ dst)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t per_mat = (size_t)rows * nsb;
    if (i >= per_mat * mats) return;
    const int m = (int)(i / per_mat);
    const size_t j = i - (size_t)m * per_mat;
    const int r = (int)(j / nsb), sb = (int)(j % nsb);
    const uint8_t *in = src + (size_t)m * nb2 + (size_t)r * nb1 + (size_t)sb * Q8_STEP_ROW;
    uint8_t *run = dst + (size_t)m * rows * nsb * Q8_STEP_ROW + ((size_t)(r / 16) * nsb + sb) * Q8_TILE;
    const int r16 = r % 16;
    uint8_t piece[16];
    // piece 0: the eight scales
#pragma unroll
    for (int b = 0; b < 8; b++) {
        piece[2 * b] = in[b * Q8_0_BYTES];
        piece[2 * b + 1] = in[b * Q8_0_BYTES + 1];
    }
    *reinterpret_cast<uint4 *>(run + r16 * 16) = *reinterpret_cast<const uint4 *>(piece);
    // pieces 1 + 4g + t: group g's bytes 16t .. 16t + 15 = blocks 2t, 2t + 1
#pragma unroll
    for (int g = 0; g < 4; g++)
#pragma unroll
        for (int t = 0; t < 4; t++) {
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int b = 0; b < 8; b++) piece[8 * h + b] = in[(2 * t + h) * Q8_0_BYTES + 2 + 8 * g + b];
            *reinterpret_cast<uint4 *>(run + ((1 + 4 * g + t) * 16 + r16) * 16) =
                *reinterpret_cast<const uint4 *>(piece);
        }
}

hipError_t launch_tile_q80(const uint8_t *src, size_t nb1, size_t nb2, int rows, int K, int mats,
                           uint8_t *dst, hipStream_t s)
{
    if (rows % 16 || K % 256 || (nb1 % 2) || (mats > 1 && nb2 % 2)) return hipErrorInvalidValue;
    const size_t total = (size_t)rows * (K / 256) * mats;
    hipLaunchKernelGGL(k_tile_q80, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, src, nb1, nb2,
                       rows, K / 256, mats, dst);
    return hipGetLastError();
}

// Work items of phase 0: routed (work-list entry ec, group of 256 rows), then
// shared (chunk of 8 tokens, group of 256 rows); each wavefront 16 rows of
// each 128-row half, passes gate / up of the first half, gate / up of the
// second; the epilogue converts h to the down products' layout.  Phase 1:
// groups of 256 rows, each wavefront two 16-row tiles (one per pass).  A shared
// item's 16 activation rows are the a1 / a0 digit rows of its 8 tokens
// interleaved, as in k_expert.hip.
template <int PHASE>
__global__ __launch_bounds__(Q8_WAVES * 64, 2) void k_expert_q80(MoeJob job)
{
    constexpr bool DOWN = PHASE == 1;
    constexpr int GROWS = DOWN ? Q8_GROWS_DN : Q8_GROWS_GU;
    constexpr int IT = DOWN ? Q8_IT_DN : Q8_IT_GU;
    __shared__ __align__(16) uint8_t s_act[Q8_STAGES][Q8_ABYTES];
    __shared__ __align__(16) uint8_t s_w[Q8_WAVES][Q8_STAGES][Q8_TILE];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r16 = lane & 15;
    const int N = job.n_tokens, K = job.top_k;
    const int H = job.H, FF = job.FF, SF = job.SF;
    const int n_ec = job.wl.n_ec[0];
    const int nch = job.has_shared ? (N + SHARED_CHUNK - 1) / SHARED_CHUNK : 0;
    const int rg = (DOWN ? H : FF) / GROWS, rg_sh = (DOWN ? H : SF) / GROWS;
    const int routed_items = n_ec * rg;
    const int total = routed_items + nch * rg_sh;
    const int Kin = DOWN ? FF : H;                   // reduction length (SF == FF when shared)
    const int nsb = Kin / 256;
    const int steps = IT * nsb;
    const uint32_t act_base = q8_lds_addr(&s_act[0][0]);
    const uint32_t w_base = q8_lds_addr(&s_w[wave][0][0]);
    // weight load jd of a step: lane's piece p = 64 jd + lane (p < 272) of the
    // tile run, copied to slot p of the stage
    const int pmax = Q8_WPIECES - 1;
    // activation loads: wavefront w < 4: q rows 4w .. 4w+3 (16 lanes a row,
    // lane's 16-byte slot holding logical unit (lane & 15) ^ (row & 11));
    // wavefronts 4, 5: scales of blocks 0..3 / 4..7, one 4-byte lane per
    // (block, row), stored [block][row]
    const int rq = 4 * wave + (lane >> 4);
    const int aunit = (lane & 15) ^ (rq & 11);
    const int rd = lane & 15, jd0 = (wave == 5 ? 4 : 0) + (lane >> 4);
    const bool aq_on = wave < 4, ad_on = wave == 4 || wave == 5;

    for (int item = blockIdx.x; item < total; item += gridDim.x) {
        const bool shared = item >= routed_items;
        const int j = shared ? item - routed_items : item;
        const int rgn = shared ? rg_sh : rg;
        const int unit = j / rgn;
        const int rbase = (j - unit * rgn) * GROWS;
        int t_first, nt, e = 0;
        if (!shared) {
            e = job.wl.ec_expert[unit];
            const int c0 = job.wl.ec_chunk[unit] * EXPERT_CHUNK;
            t_first = job.offsets[e] + c0;
            nt = min(EXPERT_CHUNK, job.counts[e] - c0);
        } else {
            t_first = unit * SHARED_CHUNK;
            nt = min(SHARED_CHUNK, N - t_first);
        }
        // this wavefront's tile of pass it: tb[it]
        const uint8_t *tb[IT];
        if (!DOWN) {
            const WTensor &a = shared ? job.sg : job.eg;
            const WTensor &b = shared ? job.su : job.eu;
#pragma unroll
            for (int p = 0; p < IT; p++) {
                const int t16 = (rbase + 128 * (p >> 1)) / 16 + wave;
                const WTensor &w = (p & 1) ? b : a;
                tb[p] = w.data + (size_t)e * w.nb2 + (size_t)t16 * nsb * Q8_TILE;
            }
        } else {
            const WTensor &a = shared ? job.sd : job.ed;
            const int t16 = rbase / 16 + 2 * wave;
            tb[0] = a.data + (size_t)e * a.nb2 + (size_t)t16 * nsb * Q8_TILE;
            tb[1] = tb[0] + (size_t)nsb * Q8_TILE;
        }
        const ActI8 &act = DOWN ? (shared ? job.ahs : job.ah) : (shared ? job.axs : job.ax);
        auto act_row = [&](int r) -> int {
            if (shared) return t_first + min(r >> 1, nt - 1) + (r & 1) * N;
            const int p = job.perm[t_first + min(r, nt - 1)];
            return DOWN ? p : p / K;
        };
        const int8_t *aq = act.q;
        const float *ad = act.d;
        if (aq_on) aq += (size_t)act_row(rq) * Kin + aunit * 16;
        if (ad_on) ad += (size_t)act_row(rd) * (Kin / 32) + jd0;

        // step s (pass s / nsb, 256-value step s % nsb): the wavefront's tile
        // run into its ring stage, its activation loads into the workgroup's
        // pass of step s and its 256-value step (no division: at most 3 passes
        // to skip)
        auto pass_of = [&](int s, int &sb) -> int {
            int it = 0;
            sb = s;
#pragma unroll
            for (int q = 1; q < IT; q++)
                if (sb >= nsb) { sb -= nsb; it++; }
            return it;
        };
        auto issue = [&](int s) {
            if (s >= steps) return;
            int sb;
            const int it = pass_of(s, sb);
            const int stg = s % Q8_STAGES;
            const uint8_t *t0 = tb[0];
#pragma unroll
            for (int q = 1; q < IT; q++)
                if (it == q) t0 = tb[q];
            const uint8_t *run = t0 + (size_t)sb * Q8_TILE;
            const uint32_t wst = w_base + (uint32_t)(stg * Q8_TILE);
#pragma unroll
            for (int jd = 0; jd < Q8_WDMA; jd++) {
                const int p = min(64 * jd + lane, pmax);
                if (64 * (jd + 1) <= Q8_WPIECES || 64 * jd + lane < Q8_WPIECES)
                    q8_lds_load16_nt(run + p * 16, wst + 1024 * jd);
            }
            const uint32_t ast = act_base + (uint32_t)(stg * Q8_ABYTES);
            if (aq_on) q8_lds_load16(aq + sb * 256, ast + 1024 * wave);
            if (ad_on) q8_lds_load4(ad + sb * 8, ast + Q8_AD_OFF + (wave == 5 ? 256 : 0));
        };

        // the previous item's reads of the rings are done in every wavefront
        Q8_WAIT_VM(0);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int s = 0; s < Q8_STAGES - 1; s++) issue(s);

        float acc[IT][4];
#pragma unroll
        for (int it = 0; it < IT; it++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[it][i] = 0.0f;
        for (int s = 0; s < steps; s++) {
            // step s's loads have landed once the later step's are all that may
            // be in flight (Q8_WDMA loads per step, plus one in wavefronts
            // 0..5); in the last step: wait for all.  The barrier makes that
            // true of every wavefront and frees the stages read in step s - 1.
            if (s + Q8_STAGES - 2 < steps) {
                if (wave < 6)
                    Q8_WAIT_VM((Q8_WDMA + 1) * (Q8_STAGES - 2));
                else
                    Q8_WAIT_VM(Q8_WDMA * (Q8_STAGES - 2));
            } else {
                Q8_WAIT_VM(0);
            }
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            issue(s + Q8_STAGES - 1);
            int sbc;
            const int it = pass_of(s, sbc);
            const int stg = s % Q8_STAGES;
            const uint4 *wt = reinterpret_cast<const uint4 *>(&s_w[wave][stg][0]);
            const uint8_t *ast = s_act[stg];
            // weight operands: scales (piece 0) and lane group g's 64 quant bytes
            const uint4 wd = wt[r16];
            const uint4 w01 = wt[(1 + 4 * g) * 16 + r16], w23 = wt[(2 + 4 * g) * 16 + r16];
            const uint4 w45 = wt[(3 + 4 * g) * 16 + r16], w67 = wt[(4 + 4 * g) * 16 + r16];
            long a[8], w[8];
            q80_act_ops(ast, r16, g, a);
            q80_w_ops(w01, w23, w45, w67, w);
            float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            q80_products(a, w, wd, ast, g, sum);
#pragma unroll
            for (int q = 0; q < IT; q++)
                if (it == q)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[q][i] += sum[i];
        }

        if (!DOWN) {
            // h = silu(gate) * up for the item's activation rows and its 256
            // moe_ff rows, converted in place to the down products' operand
            // layout (routed: Q8_0, shared: two int8 digits per 32 values;
            // dmoe_prep.h).  No loads are in flight after the last step: h
            // goes through the weight-ring LDS, the conversion scratch through
            // the activation ring's.
            float *s_h = reinterpret_cast<float *>(&s_w[0][0][0]);      // [16][256]
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const int col = 128 * hh + 16 * wave + r16;
                if (!shared) {
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        s_h[(4 * g + i) * 256 + col] = q8_silu(acc[2 * hh][i]) * acc[2 * hh + 1][i];
                } else {
#pragma unroll
                    for (int i = 0; i < 4; i += 2)
                        s_h[(2 * g + (i >> 1)) * 256 + col] = q8_silu(acc[2 * hh][i] + acc[2 * hh][i + 1]) *
                                                              (acc[2 * hh + 1][i] + acc[2 * hh + 1][i + 1]);
                }
            }
            __syncthreads();
            float *sv = reinterpret_cast<float *>(&s_act[0][0]) + wave * 256;
            const int sb = rbase / 256, nsb_h = (shared ? SF : FF) / 256;
            for (int t = wave; t < nt; t += Q8_WAVES) {
                float v[4];
#pragma unroll
                for (int c = 0; c < 4; c++) v[c] = s_h[t * 256 + lane + 64 * c];
                if (!shared)
                    prep_values(v, job.ah, ACT_Q80, job.perm[t_first + t], N * K, sb, nsb_h, sv);
                else
                    prep_values(v, job.ahs, ACT_SPLIT32, t_first + t, N, sb, nsb_h, sv);
            }
            continue;
        }

        // results of the down products
        float *out = shared ? job.ys : job.ye;
        const int row0 = rbase + 32 * wave;
        if (!shared) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                if (4 * g + i >= nt) continue;
                float *o = out + (size_t)job.perm[t_first + 4 * g + i] * H + row0 + r16;
                o[0] = acc[0][i];
                o[16] = acc[1][i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
                if (2 * g + (i >> 1) >= nt) continue;
                float *o = out + (size_t)(t_first + 2 * g + (i >> 1)) * H + row0 + r16;
                o[0] = acc[0][i] + acc[0][i + 1];
                o[16] = acc[1][i] + acc[1][i + 1];
            }
        }
    }
}

int expert_q80_rows_per_item(int phase) { return phase == 0 ? Q8_GROWS_GU : Q8_GROWS_DN; }

hipError_t launch_expert_q80(int phase, const MoeJob &job, hipStream_t s)
{
    if (job.FF % Q8_GROWS_GU || job.FF % 256 || job.H % Q8_GROWS_DN || job.H % 256 ||
        job.ax.K != job.H || job.ah.K != job.FF ||
        (job.has_shared && (job.SF != job.FF || job.ahs.K != job.SF)))
        return hipErrorInvalidValue;
    if (phase == 0)
        hipLaunchKernelGGL(k_expert_q80<0>, dim3(Q8_BLOCKS), dim3(Q8_WAVES * 64), 0, s, job);
    else
        hipLaunchKernelGGL(k_expert_q80<1>, dim3(Q8_BLOCKS), dim3(Q8_WAVES * 64), 0, s, job);
    return hipGetLastError();
}

} // namespace dmoe
