// k_expert.hip — grouped Q4_K expert products on int8 MFMA (gfx950).
//
// Computes the routed experts of src/diffuse-moe-graph.cpp:264-269 (ggml's
// mul_mat_id over Q4_K weights with Q8_K activations) and the shared expert of
// :280-286 (F32 activations, here two int8 digits), as one persistent launch
// per phase:
//   phase 0: h = silu(W_gate x) * (W_up x)       (gate and up of the same rows)
//   phase 1: y = W_down h
// (the conversion of h to the int8 layout runs in between, k_prep.hip).
//
// Arithmetic.  A Q4_K row is, per 256-value super-block, w = d*sc_j*q - dmin*m_j
// (j = 32-value sub-block, q in 0..15, sc_j, m_j 6-bit).  With int8
// activations a and their scale d_x this is ggml's vec_dot_q4_K_q8_K:
//   sum_k w a = d * sum_j sc_j S_j - dmin * sum_j m_j B_j,
//   S_j = sum_{k in j} q_k a_k (int32),  B_j = sum_{k in j} a_k.
// S_j comes from one v_mfma_i32_16x16x32_i8 per sub-block (the nibbles are the
// int8 operand), sum_j sc_j S_j from integer multiply-adds (exact), the min
// term from v_mfma_f32_16x16x16_f16 on the sums of 16 (exact integers in f16).
// The super-block result is scaled by d_x and accumulated in f32.
//
// Operand layout (checked on the hardware): srcA lane l = activation row l%16,
// k = 8*(l/16) + byte; srcB lane l = weight row l%16, same k; D lane l = weight
// row l%16, activation rows 4*(l/16)+i.  The tiled weight layout (k_quant.hip)
// puts the 32 quant bytes lane group g needs (bytes 32c + 8g .. +8 of each
// 32-byte chunk c: low nibbles = sub-block 2c, high = 2c+1) side by side, and
// repacks the 6-bit scales so that each is one bit-field extract.
//
// Memory.  A workgroup's eight wavefronts share one work item (16 activation
// rows).  Per step (one super-block) each wavefront copies its own weight
// tiles (contiguous 2304-byte runs) into a private ring of LDS stages, and six
// of them copy the step's activations into the workgroup's activation ring,
// with LDS-direct loads (global_load_lds_dwordx4): two steps stay in flight
// without holding registers.
#include "dmoe_q4k.h"

#include <cstdlib>
#include <type_traits>

namespace dmoe {


// Tuning constants (overridable at compile time).
#ifndef DMOE_X_WSTAGES
#define DMOE_X_WSTAGES 3         // LDS stages of each wavefront's weight ring
#endif
#ifndef DMOE_X_DN_IT
#define DMOE_X_DN_IT 2           // row passes of a down item (shared activation tile)
#endif
#ifndef DMOE_X_BLOCKS
#define DMOE_X_BLOCKS 1024       // persistent grid
#endif
#ifndef DMOE_X_WAVES
#define DMOE_X_WAVES 8           // wavefronts per workgroup (one workgroup per CU)
#endif
constexpr int WAVES = DMOE_X_WAVES;
constexpr int RT = 2;                        // 16-row weight tiles per wave per step
constexpr int WSTAGES = DMOE_X_WSTAGES;
constexpr int DN_IT = DMOE_X_DN_IT;
static_assert(DN_IT >= 1 && DN_IT <= 4, "row passes of a down item");
constexpr int GU_IT = 2;                         // row passes of a gate/up item
constexpr int GROWS_GU = WAVES * 16 * GU_IT;     // gate/up rows of an item: one h super-block
constexpr int GROWS_DN = WAVES * 16 * RT * DN_IT;   // down rows of an item
constexpr int WSTEP_BYTES = RT * TILE_BYTES;             // one wave's weights of one step
constexpr int WLOADS = RT * 3;                           // LDS-direct loads per step: 64 + 64 + 16 pieces a tile

// Work items of phase 0: routed (work-list entry ec, group of GROWS_GU rows),
// then shared (chunk of 8 NC tokens, group of GROWS_GU rows); phase 1 the
// same with groups of GROWS_DN rows.  A routed item's activation rows are the
// pairs of its entry (one expert, up to 16 NC consecutive pairs of it, in NC
// column blocks of 16); a shared item's are the a1 / a0 digit rows of its
// tokens interleaved (t a1, t a0, ...; 8 tokens per column block), so that
// each lane's four outputs are (t, a1), (t, a0), (t+1, a1), (t+1, a0) and the
// two digits' products are summed in-lane.  NC > 1 (many tokens per expert)
// multiplies every weight tile read from HBM by NC activation blocks: the
// weights stream once per 16 NC pairs instead of once per 16.
//
// Step s of an item is super-block s % nsb of row pass s / nsb.  Its weights
// (each wavefront's own tiles) and its activations (the workgroup's 16 NC
// rows, loaded by wavefronts 0..5) go to ring stage s % WST with LDS-direct
// loads issued WST - 1 steps ahead; one barrier per step makes the
// activations visible to all wavefronts and frees the stage for refilling.
template <int PHASE, int NC>
__global__ __launch_bounds__(WAVES * 64, 2) void k_expert_q4k(MoeJob job)
{
    constexpr bool DOWN = PHASE == 1;
    // row passes per item (a down item of 4 column blocks takes one, which
    // keeps its accumulators and two items' pointers in registers)
    constexpr int IT = DOWN ? (NC >= 4 ? 1 : DN_IT) : GU_IT;
    constexpr int GROWS = DOWN ? WAVES * 16 * RT * IT : GROWS_GU;
    // ring depths: one column block runs both rings WSTAGES deep, loads of
    // a step issued together WSTAGES - 1 steps ahead; NC > 1 blocks keep the
    // weight ring three deep (two steps of HBM loads in flight) and the
    // activation ring two deep (its loads come from L2, one step ahead), which
    // is what the LDS holds next to NC activation blocks per stage
    // Gate/up items of one column block run the weight ring four deep (three
    // steps of HBM loads in flight) beside a three-deep activation ring whose
    // loads (from L2) go two steps ahead, issued before the weights of the
    // step after: 161,472 bytes of LDS.
    constexpr bool SPLIT = !DOWN && NC == 1;
    constexpr int WST = SPLIT ? 4 : NC == 1 ? WSTAGES : 3;   // weight ring
    constexpr int AST = SPLIT ? 3 : NC == 1 ? WSTAGES : 2;   // activation ring
    constexpr int CH = EXPERT_CHUNK * NC;            // pairs of a routed item
    constexpr int SCH = SHARED_CHUNK * NC;           // tokens of a shared item
    __shared__ __align__(16) uint8_t s_act[AST][NC * ASTEP_BYTES];
    __shared__ __align__(16) uint8_t s_w[WAVES][WST][WSTEP_BYTES];
    static_assert(NC * 16 * 256 * 4 <= WAVES * WST * WSTEP_BYTES, "h of a gate/up item fits the weight ring");
    static_assert(WAVES * 256 * 4 <= AST * NC * ASTEP_BYTES, "conversion scratch fits the activation ring");
    static_assert(NC == 1 || (WST == 3 && AST == 2), "the NC > 1 issue order below assumes these depths");

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const int N = job.n_tokens, K = job.top_k;
    const int H = job.H, FF = job.FF, SF = job.SF;
    const int n_ec = job.wl.n_ec[0];
    const int nch = job.has_shared ? (N + SCH - 1) / SCH : 0;
    const int rg = (DOWN ? H : FF) / GROWS, rg_sh = (DOWN ? H : SF) / GROWS;
    const int routed_items = n_ec * rg;
    const int total = routed_items + nch * rg_sh;
    const int Kin = DOWN ? FF : H;                   // reduction length (SF == FF when shared)
    const int nsb = Kin / 256;
    const int steps = IT * nsb;
    // weight loads of a step: tile r's pieces 64 j + lane (j = 0, 1, and 2 for
    // lanes below TPIECES - 128) from the tile's step run, to slot 64 j + lane
    // of the tile's place in the stage
    const uint32_t loff = lane * 16;
    // activation load of this wavefront (wavefronts 0..5): which block row
    // (ar) and piece; 0..3: q units of rows 4w .. 4w+3, 4: bs halves, 5: d
    const int ar = wave < 4 ? 4 * wave + (lane >> 4) : (wave == 4 ? (lane >> 1) & 15 : lane & 15);
    const int aunit = (lane & 15) ^ (ar & 11);       // q: logical unit of this lane's slot
    const bool aload = wave < 4 || (wave == 4 && lane < 32) || (wave == 5 && lane < 16);

    // The pointers of one work item.
    struct ItemPtrs {
        const uint8_t *tb[IT][RT];   // this wave's weight tiles of pass it
        const int8_t *aq[NC];        // the lane's activation load sources, per block
        const uint16_t *abs_[NC];
        const float *ad[NC];
        int t_first, nt, rbase, nblk;
        bool shared;
    };
    auto setup = [&](int item, ItemPtrs &P) {
        const bool shared = item >= routed_items;
        const int j = shared ? item - routed_items : item;
        const int rgn = shared ? rg_sh : rg;
        const int unit = j / rgn;                 // work-list entry or shared chunk
        const int rbase = (j - unit * rgn) * GROWS;
        int t_first, nt, e = 0;
        if (!shared) {
            e = job.wl.ec_expert[unit];
            const int c0 = job.wl.ec_chunk[unit] * CH;
            t_first = job.offsets[e] + c0;
            nt = min(CH, job.counts[e] - c0);
        } else {
            t_first = unit * SCH;
            nt = min(SCH, N - t_first);
        }
        if (!DOWN) {
            const WTensor &a = shared ? job.sg : job.eg;
            const WTensor &b = shared ? job.su : job.eu;
#pragma unroll
            for (int it = 0; it < IT; it++) {
                const int t16 = (rbase + it * (WAVES * 16) + wave * 16) / 16;
                P.tb[it][0] = a.data + (size_t)e * a.nb2 + (size_t)t16 * nsb * TILE_BYTES;
                P.tb[it][1] = b.data + (size_t)e * b.nb2 + (size_t)t16 * nsb * TILE_BYTES;
            }
        } else {
            const WTensor &a = shared ? job.sd : job.ed;
#pragma unroll
            for (int it = 0; it < IT; it++)
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    const int t16 = (rbase + it * (WAVES * 32) + wave * 32) / 16 + r;
                    P.tb[it][r] = a.data + (size_t)e * a.nb2 + (size_t)t16 * nsb * TILE_BYTES;
                }
        }
        // the activation row of block row ar of each block: tokens in phase
        // 0, pairs in phase 1; shared rows interleave the a1 and a0 digit
        // rows (a0 rows start at N).  Rows past the item's last repeat it (a
        // block past it loads the last row again and is not computed).
        const ActI8 &act = DOWN ? (shared ? job.ahs : job.ah) : (shared ? job.axs : job.ax);
        const int per = shared ? SHARED_CHUNK : EXPERT_CHUNK;   // items of a block
#pragma unroll
        for (int c = 0; c < NC; c++) {
            int arow;
            if (shared) {
                arow = t_first + min(per * c + (ar >> 1), nt - 1) + (ar & 1) * N;
            } else {
                const int p = job.perm[t_first + min(per * c + ar, nt - 1)];
                arow = DOWN ? p : p / K;
            }
            P.aq[c] = act.q + (size_t)arow * Kin + aunit * 16;
            P.abs_[c] = act.bs + (size_t)arow * (Kin / 16) + (lane & 1) * 8;
            P.ad[c] = act.d + (size_t)arow * nsb;
        }
        P.t_first = t_first;
        P.nt = nt;
        P.rbase = rbase;
        P.nblk = (nt + per - 1) / per;
        P.shared = shared;
    };

    // row pass of step s (at most four passes: no division)
    auto pass_of = [&](int s) -> int {
        int it = 0;
#pragma unroll
        for (int q = 1; q < IT; q++) it += s >= q * nsb ? 1 : 0;
        return it;
    };
    // weights of step s of item P to weight stage gstep % WST
    auto issue_w = [&](const ItemPtrs &P, int s, int gstep) {
        if (s >= steps) return;
        const int it = pass_of(s), sb = s - it * nsb;
        const int stg = gstep % WST;
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const uint8_t *t = P.tb[0][r];
#pragma unroll
            for (int q = 1; q < IT; q++)
                if (it == q) t = P.tb[q][r];
            t += (size_t)sb * TILE_BYTES;
            const uint8_t *d = &s_w[wave][stg][r * TILE_BYTES];
            lds_load16_sa(t, loff, d);
            lds_load16_sa(t, loff + 1024, d + 1024);
            if (lane < TPIECES - 128) lds_load16_sa(t, loff + 2048, d + 2048);
        }
    };
    // activations of step s of item P to activation stage gstep % AST
    auto issue_a = [&](const ItemPtrs &P, int s, int gstep) {
        if (s >= steps) return;
        const int it = pass_of(s), sb = s - it * nsb;
        const int stg = gstep % AST;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            uint8_t *st = &s_act[stg][c * ASTEP_BYTES];
            if (wave < 4)
                lds_load16(P.aq[c] + sb * 256, st + 1024 * wave);
            else if (wave == 4 && aload)
                lds_load16(P.abs_[c] + sb * 16, st + ABS_OFF);
            else if (wave == 5 && aload)
                lds_load4(P.ad[c] + sb, st + AD_OFF);
        }
    };
    // both parts of step s (the one-block order: weights, then activations)
    auto issue = [&](const ItemPtrs &P, int s, int gstep) {
        issue_w(P, s, gstep);
        issue_a(P, s, gstep);
    };

    // Down items end with global stores only, so the rings run on from one
    // item of this workgroup to its next: the last steps of an item issue
    // the next item's first WST - 1 steps (ring positions continue), and
    // the next item starts without draining.  Gate/up items convert h through
    // the rings after their last step, so each starts from drained rings.
    constexpr bool XPF = DOWN;
    ItemPtrs cur, nx;
    bool primed = false;             // cur's first WST - 1 steps are issued
    int g0 = 0;                      // ring position of cur's step 0
    for (int item = blockIdx.x; item < total; item += gridDim.x) {
        if (primed)
            cur = nx;
        else
            setup(item, cur);
        const int nitem = item + gridDim.x;
        const bool has_next = XPF && steps >= 2 && nitem < total;
        if (has_next) setup(nitem, nx);
        const bool shared = cur.shared;
        const int t_first = cur.t_first, nt = cur.nt, rbase = cur.rbase, nblk = cur.nblk;

        if (!primed) {
            // the previous item's reads of the rings are done in every wavefront
            g0 = 0;
            EXPERT_WAIT_VM(0);
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if constexpr (SPLIT) {
                // W(0), A(0), W(1), A(1), W(2): the steady order A(s + 2), W(s + 3)
                issue_w(cur, 0, 0);
                issue_a(cur, 0, 0);
                issue_w(cur, 1, 1);
                issue_a(cur, 1, 1);
                issue_w(cur, 2, 2);
            } else if constexpr (NC == 1) {
#pragma unroll
                for (int s = 0; s < WST - 1; s++) issue(cur, s, s);
            } else {
                // W(0), A(0), W(1): step 0 waits with only W(1) in flight
                issue_w(cur, 0, 0);
                issue_a(cur, 0, 0);
                issue_w(cur, 1, 1);
            }
        }

        float acc[IT][NC][RT][4];
#pragma unroll
        for (int it = 0; it < IT; it++)
#pragma unroll
            for (int c = 0; c < NC; c++)
#pragma unroll
                for (int r = 0; r < RT; r++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[it][c][r][i] = 0.0f;
        for (int s = 0; s < steps; s++) {
            // step s's loads have landed once the WST - 2 later steps' are
            // all that may be in flight (a wavefront issues WLOADS loads per step,
            // plus NC when it loads activations; the previous item's output
            // stores, when they follow, only make this stricter); when fewer
            // later steps were issued (the item's last steps, no next item
            // primed): wait for all.  The barrier makes that true of every
            // wavefront and frees the stage read in the step before.
            if constexpr (SPLIT) {
                // A(s) was issued after W(s); after it: W(s + 1), A(s + 1),
                // W(s + 2), those of them that exist
                const int al = wave < ADMA_WAVES ? 1 : 0;
                if (s + 2 < steps) {
                    if (al)
                        EXPERT_WAIT_VM(2 * WLOADS + 1);
                    else
                        EXPERT_WAIT_VM(2 * WLOADS);
                } else if (s + 1 < steps) {
                    if (al)
                        EXPERT_WAIT_VM(WLOADS + 1);
                    else
                        EXPERT_WAIT_VM(WLOADS);
                } else {
                    EXPERT_WAIT_VM(0);
                }
            } else if constexpr (NC == 1) {
                if (s + WST - 2 < steps || has_next) {
                    if (wave < ADMA_WAVES)
                        EXPERT_WAIT_VM((WLOADS + 1) * (WST - 2));
                    else
                        EXPERT_WAIT_VM(WLOADS * (WST - 2));
                } else {
                    EXPERT_WAIT_VM(0);
                }
            } else {
                // issue order per step: A(s + 1), then W(s + 2); so when
                // step s runs only W(s + 1) may still be in flight (every
                // earlier load, A(s) included, was issued before it)
                if (s + 1 < steps || has_next)
                    EXPERT_WAIT_VM(WLOADS);
                else
                    EXPERT_WAIT_VM(0);
            }
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if constexpr (SPLIT) {
                if (s + 2 < steps) issue_a(cur, s + 2, s + 2);
                if (s + 3 < steps) issue_w(cur, s + 3, s + 3);
            } else if constexpr (NC == 1) {
                const int sn = s + WST - 1;
                if (sn < steps)
                    issue(cur, sn, g0 + sn);
                else if (has_next)
                    issue(nx, sn - steps, g0 + sn);
            } else {
                const int sa = s + 1, sw = s + 2;
                if (sa < steps)
                    issue_a(cur, sa, g0 + sa);
                else if (has_next)
                    issue_a(nx, sa - steps, g0 + sa);
                if (sw < steps)
                    issue_w(cur, sw, g0 + sw);
                else if (has_next)
                    issue_w(nx, sw - steps, g0 + sw);
            }
            const int it = pass_of(s);
            const int stg = (g0 + s) % WST, astg = (g0 + s) % AST;
            if constexpr (NC == 1) {
                Q4KTile cur_t[RT];
#pragma unroll
                for (int r = 0; r < RT; r++) read_tile(cur_t[r], &s_w[wave][stg][r * TILE_BYTES], r16, g);
#pragma unroll
                for (int q = 0; q < IT; q++)
                    if (it == q) compute_sb(cur_t, s_act[astg], r16, g, acc[q][0]);
            } else {
                // each tile's operands formed once, then every column block
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    Q4KTile t;
                    read_tile(t, &s_w[wave][stg][r * TILE_BYTES], r16, g);
                    Q4KFolded f;
                    fold_tile(t, g, f);
#pragma unroll
                    for (int c = 0; c < NC; c++)
                        if (c < nblk)
#pragma unroll
                            for (int q = 0; q < IT; q++)
                                if (it == q) compute_folded(f, &s_act[astg][c * ASTEP_BYTES], r16, g, acc[q][c][r]);
                }
            }
        }
        primed = has_next;
        g0 += steps;

        if (!DOWN) {
            // h = silu(gate) * up for the item's activation rows and its 256
            // moe_ff rows (one super-block), then converted in place to the
            // down products' operand layout (routed: Q8_K, shared: two int8
            // digits; dmoe_prep.h) -- no f32 h in HBM.  The rings are idle
            // (no loads in flight after the last step): h goes through the
            // weight-ring LDS, the conversion scratch through the activation
            // ring's.
            float *s_h = reinterpret_cast<float *>(&s_w[0][0][0]);      // [16 NC][256]
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
#pragma unroll
            for (int it = 0; it < IT; it++) {
                const int col = it * (WAVES * 16) + wave * 16 + r16;
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    if (c >= nblk) continue;
                    if (!shared) {
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            s_h[(16 * c + 4 * g + i) * 256 + col] = silu(acc[it][c][0][i]) * acc[it][c][1][i];
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; i += 2)
                            s_h[(8 * c + 2 * g + (i >> 1)) * 256 + col] =
                                silu(acc[it][c][0][i] + acc[it][c][0][i + 1]) *
                                (acc[it][c][1][i] + acc[it][c][1][i + 1]);
                    }
                }
            }
            __syncthreads();
            float *sv = reinterpret_cast<float *>(&s_act[0][0]) + wave * 256;
            const int sb = rbase / 256, nsb_h = (shared ? SF : FF) / 256;
            for (int t = wave; t < nt; t += WAVES) {
                float v[4];
#pragma unroll
                for (int c = 0; c < 4; c++) v[c] = s_h[t * 256 + lane + 64 * c];
                if (!shared)
                    prep_values(v, job.ah, ACT_Q8K, job.perm[t_first + t], N * K, sb, nsb_h, sv);
                else
                    prep_values(v, job.ahs, ACT_SPLIT, t_first + t, N, sb, nsb_h, sv);
            }
            continue;
        }

        // results of the down products
        float *out = shared ? job.ys : job.ye;
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int row0 = rbase + it * (WAVES * 32) + wave * 32;
#pragma unroll
            for (int c = 0; c < NC; c++) {
                if (c >= nblk) continue;
                if (!shared) {
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int q = 16 * c + 4 * g + i;
                        if (q >= nt) continue;
                        float *o = out + (size_t)job.perm[t_first + q] * H + row0 + r16;
#pragma unroll
                        for (int r = 0; r < RT; r++) o[16 * r] = acc[it][c][r][i];
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 4; i += 2) {
                        const int q = 8 * c + 2 * g + (i >> 1);
                        if (q >= nt) continue;
                        float *o = out + (size_t)(t_first + q) * H + row0 + r16;
#pragma unroll
                        for (int r = 0; r < RT; r++) o[16 * r] = acc[it][c][r][i] + acc[it][c][r][i + 1];
                    }
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Gate/up items of one column block (few tokens) with the weights streamed to
// registers: the same items, rows and arithmetic as k_expert_q4k<0, 1>, but
// the item's activations (16 rows of every super-block, 74.75 KB at n_embd
// 4096) are loaded into LDS once at the item's start and each wavefront
// streams its gate and up tiles to a ring of GR_R register sets, GR_R - 1
// steps ahead (the compiler's own loads: its waits are exact), with no
// barrier in the step loop.  The first steps' weights are issued before the
// item's pairs and activation rows are looked up.  The h conversion after
// the last step is k_expert_q4k's, through the activation region.  The
// stream is bandwidth bound in the steady state: more register sets only
// lengthen the ramp (kernel trace at 32 tokens: 45.1, 46.1, 47.0, 47.3 us for
// 2, 3, 4, 5 sets; 171 / 174 us for 2 / 3 sets at 256 tokens).
constexpr int GR_R = 2;          // weight register sets per wavefront (one step ahead)
constexpr int GR_MAX_SB = 16;    // super-blocks of the reduction held in LDS (n_embd <= 4096)
constexpr int GR_TAB_E = 1024;   // routed experts whose offsets and counts are staged in LDS
constexpr int GR_TAB_P = 2048;   // (token, slot) pairs whose permutation entries are staged

template <int J0, int J1, class F>
__device__ __forceinline__ void gr_unroll(F &&f)
{
    if constexpr (J0 < J1) {
        f(std::integral_constant<int, J0>());
        gr_unroll<J0 + 1, J1>(f);
    }
}

typedef unsigned int gr_u4v __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) gr_u4v *gr_gu4v_ptr;

__device__ __forceinline__ uint4 gr_ld_nt16(const void *p)
{
    const gr_u4v v = __builtin_nontemporal_load((gr_gu4v_ptr)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// TABS: the routing's offsets, counts and permutation fit the LDS tables
// (gr_tabs) and are read from there
template <bool TABS>
__global__ __launch_bounds__(WAVES * 64) void k_gateup_rr(MoeJob job)
{
    __shared__ __align__(16) uint8_t s_act[GR_MAX_SB][ASTEP_BYTES];
    __shared__ int32_t s_off[GR_TAB_E], s_cnt[GR_TAB_E], s_perm[GR_TAB_P];
    static_assert(GROWS_GU * 16 * 4 + WAVES * 256 * 4 <= GR_MAX_SB * ASTEP_BYTES, "h and its scratch fit");

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const int N = job.n_tokens, K = job.top_k;
    const int H = job.H, FF = job.FF, SF = job.SF;
    const int rg = FF / GROWS_GU, rg_sh = SF / GROWS_GU;
    // The work-list count, the first item's work-list entry (read as if the
    // item were routed) and the routing's offsets, counts and permutation
    // (into LDS) are independent loads, issued together: one round trip
    // before the item's weight and activation addresses are known, where
    // looking them up in turn (count, entry, offset, pair) takes four.
    constexpr bool tabs = TABS;
    const int n_ec = job.wl.n_ec[0];
    int e_first = 0, c_first = 0;
    if (job.ec_cap > 0) {
        const int u = min((int)blockIdx.x / rg, job.ec_cap - 1);
        e_first = job.wl.ec_expert[u];
        c_first = job.wl.ec_chunk[u];
    }
    if constexpr (tabs) {
        for (int i = tid; i < job.E; i += WAVES * 64) {
            s_off[i] = job.offsets[i];
            s_cnt[i] = job.counts[i];
        }
        for (int i = tid; i < N * K; i += WAVES * 64) s_perm[i] = job.perm[i];
    }
    __syncthreads();
    const int nch = job.has_shared ? (N + SHARED_CHUNK - 1) / SHARED_CHUNK : 0;
    const int routed_items = n_ec * rg;
    const int total = routed_items + nch * rg_sh;
    const int nsb = H / 256;
    const int steps = GU_IT * nsb;
    // activation loads (k_expert_q4k's roles)
    const int ar = wave < 4 ? 4 * wave + (lane >> 4) : (wave == 4 ? (lane >> 1) & 15 : lane & 15);
    const int aunit = (lane & 15) ^ (ar & 11);
    const bool aload = wave < 4 || (wave == 4 && lane < 32) || (wave == 5 && lane < 16);

    for (int item = blockIdx.x; item < total; item += gridDim.x) {
        const bool shared = item >= routed_items;
        const int j = shared ? item - routed_items : item;
        const int rgn = shared ? rg_sh : rg;
        const int unit = j / rgn;
        const int rbase = (j - unit * rgn) * GROWS_GU;
        int t_first, nt, e = 0;
        if (!shared) {
            const bool first = item == (int)blockIdx.x;
            e = first ? e_first : job.wl.ec_expert[unit];
            const int c0 = (first ? c_first : job.wl.ec_chunk[unit]) * EXPERT_CHUNK;
            if constexpr (tabs) {
                t_first = s_off[e] + c0;
                nt = min(EXPERT_CHUNK, s_cnt[e] - c0);
            } else {
                t_first = job.offsets[e] + c0;
                nt = min(EXPERT_CHUNK, job.counts[e] - c0);
            }
        } else {
            t_first = unit * SHARED_CHUNK;
            nt = min(SHARED_CHUNK, N - t_first);
        }
        // this wavefront's tiles: gate and up rows rbase + 128 it + 16 wave
        const WTensor &wa = shared ? job.sg : job.eg;
        const WTensor &wb = shared ? job.su : job.eu;
        // (pass it's tiles are WAVES tiles further: no array of pointers,
        // which would be indexed from private memory)
        const int t16 = (rbase + wave * 16) / 16;
        const uint8_t *tg = wa.data + (size_t)e * wa.nb2 + (size_t)t16 * nsb * TILE_BYTES;
        const uint8_t *tu = wb.data + (size_t)e * wb.nb2 + (size_t)t16 * nsb * TILE_BYTES;
        const size_t pass_step = (size_t)WAVES * nsb * TILE_BYTES;
        // the load cursor (pass, super-block) runs GR_R - 1 steps ahead and
        // stays on the last step once there (loading it again, never used)
        int l_it = 0, l_sb = 0, lq = 0;
        auto load = [&](Q4KTile (&o)[2]) __attribute__((always_inline)) {
            const size_t off = (size_t)l_it * pass_step + (size_t)l_sb * TILE_BYTES;
            const uint4 *pg = reinterpret_cast<const uint4 *>(tg + off);
            const uint4 *pu = reinterpret_cast<const uint4 *>(tu + off);
            o[0].h = gr_ld_nt16(pg + r16);
            o[0].q0 = gr_ld_nt16(pg + (1 + 2 * g) * 16 + r16);
            o[0].q1 = gr_ld_nt16(pg + (2 + 2 * g) * 16 + r16);
            o[1].h = gr_ld_nt16(pu + r16);
            o[1].q0 = gr_ld_nt16(pu + (1 + 2 * g) * 16 + r16);
            o[1].q1 = gr_ld_nt16(pu + (2 + 2 * g) * 16 + r16);
            if (lq + 1 < steps) {
                lq++;
                if (++l_sb == nsb) {
                    l_sb = 0;
                    l_it++;
                }
            }
        };
        // this lane's activation row, looked up before the first weight loads
        // are issued (a global load after them would wait for them too)
        int arow;
        if (shared) {
            arow = t_first + min(ar >> 1, nt - 1) + (ar & 1) * N;
        } else {
            const int pi = t_first + min(ar, nt - 1);
            if constexpr (tabs)
                arow = s_perm[pi] / K;
            else
                arow = job.perm[pi] / K;
        }
        asm volatile("" : "+v"(arow));
        Q4KTile o[GR_R][2];
        gr_unroll<0, GR_R - 1>([&](auto jc) { load(o[decltype(jc)::value]); });

        // the previous item's h conversion is done with the activation region
        __syncthreads();
        const ActI8 &act = shared ? job.axs : job.ax;
        if (wave < ADMA_WAVES) {
            for (int sb = 0; sb < nsb; sb++) {
                uint8_t *st = &s_act[sb][0];
                if (wave < 4)
                    lds_load16(act.q + (size_t)arow * H + sb * 256 + aunit * 16, st + 1024 * wave);
                else if (wave == 4 && aload)
                    lds_load16(act.bs + (size_t)arow * (H / 16) + sb * 16 + (lane & 1) * 8, st + ABS_OFF);
                else if (wave == 5 && aload)
                    lds_load4(act.d + (size_t)arow * nsb + sb, st + AD_OFF);
            }
        }
        // the activation loads (and the weight loads before them) have
        // landed in every wavefront
        EXPERT_WAIT_VM(0);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");

        // the current pass's sums, and pass 0's once it is done (a register
        // copy at the pass boundary: no accumulator chosen by a run-time index)
        static_assert(GU_IT == 2, "two row passes");
        float acc[2][4], acc0[2][4];
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[r][i] = acc0[r][i] = 0.0f;
        int c_sb = 0;
        bool c_first = true;
        auto compute = [&](const Q4KTile (&w)[2]) __attribute__((always_inline)) {
            compute_sb<2>(w, &s_act[c_sb][0], r16, g, acc);
            if (++c_sb == nsb) {
                c_sb = 0;
                if (c_first) {
#pragma unroll
                    for (int r = 0; r < 2; r++)
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            acc0[r][i] = acc[r][i];
                            acc[r][i] = 0.0f;
                        }
                    c_first = false;
                }
            }
        };
        int s0 = 0;
        for (; s0 + GR_R <= steps; s0 += GR_R)
            gr_unroll<0, GR_R>([&](auto jc) {
                constexpr int jj = decltype(jc)::value;
                load(o[(jj + GR_R - 1) % GR_R]);
                compute(o[jj]);
            });
        gr_unroll<0, GR_R - 1>([&](auto jc) {
            constexpr int jj = decltype(jc)::value;
            if (s0 + jj < steps) {
                load(o[(jj + GR_R - 1) % GR_R]);
                compute(o[jj]);
            }
        });

        // h = silu(gate) * up for the item's rows, then converted to the down
        // products' operand layout (k_expert_q4k's conversion)
        float *s_h = reinterpret_cast<float *>(&s_act[0][0]);              // [16][256]
        __syncthreads();
#pragma unroll
        for (int it = 0; it < GU_IT; it++) {
            const int col = it * (WAVES * 16) + wave * 16 + r16;
            const float (&a)[2][4] = it == 0 ? acc0 : acc;
            if (!shared) {
#pragma unroll
                for (int i = 0; i < 4; i++) s_h[(4 * g + i) * 256 + col] = silu(a[0][i]) * a[1][i];
            } else {
#pragma unroll
                for (int i = 0; i < 4; i += 2)
                    s_h[(2 * g + (i >> 1)) * 256 + col] = silu(a[0][i] + a[0][i + 1]) * (a[1][i] + a[1][i + 1]);
            }
        }
        __syncthreads();
        float *sv = reinterpret_cast<float *>(&s_act[0][0]) + 16 * 256 + wave * 256;
        const int sbh = rbase / 256, nsb_h = (shared ? SF : FF) / 256;
        for (int t = wave; t < nt; t += WAVES) {
            float v[4];
#pragma unroll
            for (int c = 0; c < 4; c++) v[c] = s_h[t * 256 + lane + 64 * c];
            if (!shared)
                prep_values(v, job.ah, ACT_Q8K, tabs ? (int)s_perm[t_first + t] : (int)job.perm[t_first + t], N * K,
                            sbh, nsb_h, sv);
            else
                prep_values(v, job.ahs, ACT_SPLIT, t_first + t, N, sbh, nsb_h, sv);
        }
    }
}

int expert_rows_per_item(int phase) { return phase == 0 ? GROWS_GU : GROWS_DN; }

bool expert_k_ok(int K) { return K % 256 == 0; }

template <int PHASE>
static hipError_t launch_phase(int nc, const MoeJob &job, dim3 grid, hipStream_t s)
{
    switch (nc) {
    case 1: hipLaunchKernelGGL((k_expert_q4k<PHASE, 1>), grid, dim3(WAVES * 64), 0, s, job); break;
    case 2: hipLaunchKernelGGL((k_expert_q4k<PHASE, 2>), grid, dim3(WAVES * 64), 0, s, job); break;
    case 4: hipLaunchKernelGGL((k_expert_q4k<PHASE, 4>), grid, dim3(WAVES * 64), 0, s, job); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_expert_q4k(int phase, const MoeJob &job, hipStream_t s, int nc, bool gateup_lds)
{
    if (job.FF % GROWS_GU || job.FF % 256 || job.H % GROWS_DN || job.H % 256 ||
        job.ax.K != job.H || job.ah.K != job.FF ||
        (job.has_shared && (job.SF != job.FF || job.ahs.K != job.SF)))
        return hipErrorInvalidValue;
    // routed work-list entries hold 16 nc pairs
    if ((nc != 1 && nc != 2 && nc != 4) || (job.wl.n_ec && job.wl.chunk != EXPERT_CHUNK * nc))
        return hipErrorInvalidValue;
    if (phase == 0) {
        // one column block: the register-ring kernel unless the LDS-ring one
        // is selected (gateup_lds; the same bits)
        if (nc == 1 && job.H / 256 <= GR_MAX_SB && !gateup_lds) {
            if (job.E > 0 && job.E <= GR_TAB_E && job.n_tokens * job.top_k <= GR_TAB_P)
                hipLaunchKernelGGL(k_gateup_rr<true>, dim3(DMOE_X_BLOCKS), dim3(WAVES * 64), 0, s, job);
            else
                hipLaunchKernelGGL(k_gateup_rr<false>, dim3(DMOE_X_BLOCKS), dim3(WAVES * 64), 0, s, job);
            return hipGetLastError();
        }
        return launch_phase<0>(nc, job, dim3(DMOE_X_BLOCKS), s);
    }
    // one workgroup per compute unit (one fits at a time), so that each
    // runs its items back to back with the rings running on between them
    int n_cu = 0;
    const hipError_t e = device_cu_count(&n_cu);
    if (e != hipSuccess) return e;
    return launch_phase<1>(nc, job, dim3(n_cu), s);
}

hipError_t device_cu_count(int *out)
{
    // compute units of each device, looked up once (a repeated lookup
    // stores the same value)
    static int n_cu[64] = {0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (n_cu[dev] <= 0) {
        int n = 0;
        e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        if (n <= 0) return hipErrorInvalidDevice;
        n_cu[dev] = n;
    }
    *out = n_cu[dev];
    return hipSuccess;
}

} // namespace dmoe

