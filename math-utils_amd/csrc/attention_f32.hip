// attention_f32.hip - fp32 causal GQA attention with kernels::attention's
// semantics (include/ai/Kernels.hpp:130-168): for token t and head h at
// position start+t, keys [first, start+t] of kv head h/(heads/kvHeads), with
// first = start+t+1-window when a window is set; out = softmax(q.K/sqrt(D)) V.
//
// This is the exact-arithmetic path behind the drop-in aigpu_attention, in
// two forms. fp32 q and KV of dim 64 or 128 on 16-byte boundaries take the
// tiled form on the fp32 matrix cores (attention_f32_tile_kernel, described
// at it); every other call (bf16 KV, other dims, unaligned rows) takes the
// scalar form: fp32 loads, fp32 FMAs, expf. There one wave owns one (token,
// head) and walks the keys in blocks of 64 with an online softmax: lane j
// scores key j of the block, then the lanes switch to owning dimensions for
// the P.V accumulation. Both loops issue their loads in batches before using
// them (a key row as up to 16 16-byte pieces per lane with four partial sums
// when rows are 16-byte aligned; value rows as 16-byte pieces, several rows
// per load instruction, or else eight rows at a time), so that a block costs
// a few memory round trips rather than one per dimension or per key.
#include "context.hpp"
#include "device.hpp"
#include "kernels.hpp"

namespace aigpu {

namespace {

constexpr int MAX_DIM = 256;

__global__ __launch_bounds__(256) void attention_f32_kernel(AttentionF32Params p) {
    __shared__ __align__(16) float qs[4][MAX_DIM];
    __shared__ float ps[4][WAVE];

    const int lane = threadIdx.x & (WAVE - 1);
    const int w = threadIdx.x / WAVE;
    const uint64_t task = uint64_t(blockIdx.x) * 4 + w;
    if (task >= p.count * p.heads) return;  // whole wave leaves; no block barriers below

    const uint64_t token = task / p.heads, head = task % p.heads;
    const uint64_t position = p.start + token;
    const uint64_t first = p.window && position + 1 > p.window ? position + 1 - p.window : 0;
    const uint64_t kv = head / (p.heads / p.kvHeads);
    const int dim = int(p.dim);
    const float scale = 1.0f / sqrtf(float(dim));

    for (int d = lane; d < dim; d += WAVE)
        qs[w][d] = load_elem(p.q, (token * p.heads + head) * p.qStride + d, p.qType);
    wave_sync();

    const size_t kvBase = kv * p.headStride;
    float m = -INFINITY, l = 0.0f;
    float acc[MAX_DIM / WAVE] = {0.0f, 0.0f, 0.0f, 0.0f};
    // key rows in 16-byte pieces: every row start (and q's copy in LDS) on a
    // 16-byte boundary, which fp32 rows with dim % 4 == 0 and bf16 rows with
    // dim % 8 == 0 and strides to match give
    const size_t esz = p.kvType == 0 ? 4 : 2, per = 16 / esz;
    const bool vec = dim % int(per) == 0 && (reinterpret_cast<uintptr_t>(p.keys) % 16) == 0 &&
                     (kvBase * esz) % 16 == 0 && (p.posStride * esz) % 16 == 0;
    // fp32 value rows of dim / 4 16-byte pieces, a power of two: LPR lanes per
    // row, RPI = 64 / LPR rows per load instruction, each lane a four-float
    // accumulator for its piece and its group of rows (summed across the
    // groups at the end); up to 16 pieces per lane in flight
    const int LPR = dim / 4;
    const bool vecv = p.kvType == 0 && dim % 4 == 0 && (LPR & (LPR - 1)) == 0 &&
                      (reinterpret_cast<uintptr_t>(p.values) % 16) == 0 && (kvBase * 4) % 16 == 0 &&
                      (p.posStride * 4) % 16 == 0;
    const int RPI = vecv ? WAVE / LPR : 1, vg = vecv ? lane / LPR : 0, vc = vecv ? lane % LPR : 0;
    floatx4 acc2 = {0.0f, 0.0f, 0.0f, 0.0f};

    for (uint64_t j0 = first; j0 <= position; j0 += WAVE) {
        const uint64_t j = j0 + lane;
        const bool ok = j <= position;
        float s = -INFINITY;
        if (ok) {
            const size_t row = kvBase + j * p.posStride;
            float dot = 0.0f;
            if (vec && p.kvType == 0) {
                // up to 64 dimensions per batch: 16 pieces in flight, four partial sums
                const floatx4* kr = reinterpret_cast<const floatx4*>(static_cast<const float*>(p.keys) + row);
                const floatx4* q4 = reinterpret_cast<const floatx4*>(qs[w]);
                floatx4 part = {0.0f, 0.0f, 0.0f, 0.0f};
                for (int c0 = 0; c0 < dim / 4; c0 += 16) {
                    floatx4 kp[16];
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (c0 + i < dim / 4) kp[i] = kr[c0 + i];
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (c0 + i < dim / 4) {
                            const floatx4 qv = q4[c0 + i];
#pragma unroll
                            for (int e = 0; e < 4; ++e) part[e] = fmaf(qv[e], kp[i][e], part[e]);
                        }
                }
                dot = (part[0] + part[1]) + (part[2] + part[3]);
            } else if (vec) {
                // bf16: eight elements per piece, up to 128 dimensions per batch
                const u32x4* kr = reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p.keys) + row);
                const floatx4* q4 = reinterpret_cast<const floatx4*>(qs[w]);
                floatx4 part = {0.0f, 0.0f, 0.0f, 0.0f};
                for (int c0 = 0; c0 < dim / 8; c0 += 16) {
                    u32x4 kp[16];
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (c0 + i < dim / 8) kp[i] = kr[c0 + i];
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (c0 + i < dim / 8) {
                            const floatx4 qa = q4[2 * (c0 + i)], qb = q4[2 * (c0 + i) + 1];
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const uint32_t wv = kp[i][e];
                                const float lo = __uint_as_float(wv << 16), hi = __uint_as_float(wv & 0xFFFF0000u);
                                const float q0 = e < 2 ? qa[2 * e] : qb[2 * e - 4];
                                const float q1 = e < 2 ? qa[2 * e + 1] : qb[2 * e - 3];
                                part[e] = fmaf(q1, hi, fmaf(q0, lo, part[e]));
                            }
                        }
                }
                dot = (part[0] + part[1]) + (part[2] + part[3]);
            } else if (p.kvType == 0) {
                const float* kr = static_cast<const float*>(p.keys) + row;
                for (int d = 0; d < dim; ++d) dot = fmaf(qs[w][d], kr[d], dot);
            } else {
                const uint16_t* kr = static_cast<const uint16_t*>(p.keys) + row;
                for (int d = 0; d < dim; ++d) dot = fmaf(qs[w][d], bf16_bits_to_float(kr[d]), dot);
            }
            s = dot * scale;
        }
        const float mn = fmaxf(m, wave_max(s));  // finite: the block holds key j0
        const float alpha = expf(m - mn);
        const float pj = ok ? expf(s - mn) : 0.0f;
        l = l * alpha + wave_sum(pj);
        m = mn;
#pragma unroll
        for (int i = 0; i < MAX_DIM / WAVE; ++i) acc[i] *= alpha;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc2[e] *= alpha;

        ps[w][lane] = pj;
        wave_sync();
        const int nb = int(position + 1 - j0 < WAVE ? position + 1 - j0 : WAVE);
        if (vecv) {
            const floatx4* vb = reinterpret_cast<const floatx4*>(static_cast<const float*>(p.values) + kvBase) + vc;
            const size_t rs = p.posStride / 4;
            for (int t0 = 0; t0 < LPR; t0 += 16) {
                floatx4 vp[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const int r = (t0 + u) * RPI + vg;
                    vp[u] = t0 + u < LPR && r < nb ? vb[(j0 + uint64_t(r)) * rs] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
                }
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const int r = (t0 + u) * RPI + vg;
                    if (t0 + u < LPR && r < nb) {
                        const float pv = ps[w][r];
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc2[e] = fmaf(pv, vp[u][e], acc2[e]);
                    }
                }
            }
        }
        for (int jb = 0; !vecv && jb < nb; jb += 8) {   // eight value rows' loads in flight
            float vr[8][MAX_DIM / WAVE];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const size_t row = kvBase + (j0 + jb + u) * p.posStride;
#pragma unroll
                for (int i = 0; i < MAX_DIM / WAVE; ++i) {
                    const int d = lane + i * WAVE;
                    vr[u][i] = jb + u < nb && d < dim ? load_elem(p.values, row + d, p.kvType) : 0.0f;
                }
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (jb + u >= nb) break;   // uniform
                const float pv = ps[w][jb + u];
#pragma unroll
                for (int i = 0; i < MAX_DIM / WAVE; ++i) acc[i] = fmaf(pv, vr[u][i], acc[i]);
            }
        }
        wave_sync();
    }

    const float inv = 1.0f / l;
    float* dst = p.out + task * p.dim;
    if (vecv) {
        for (int off = LPR; off < WAVE; off <<= 1)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc2[e] += __shfl_xor(acc2[e], off, WAVE);
        if (vg == 0) {
#pragma unroll
            for (int e = 0; e < 4; ++e) dst[4 * vc + e] = acc2[e] * inv;
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < MAX_DIM / WAVE; ++i) {
        const int d = lane + i * WAVE;
        if (d < dim) dst[d] = acc[i] * inv;
    }
}

/*
    The tiled form, for fp32 q and KV of dim 64 or 128 with 16-byte aligned
    rows: the products run on the fp32 matrix cores (v_mfma_f32_32x32x2_f32
    multiplies and accumulates in fp32) and the softmax in fp32 with expf, so
    it differs from the form above only in summation order.

    A workgroup is 4 waves x 32 query tokens (TQ = 128 tokens) of one head;
    it walks key tiles of TK = 64 keys, K and V staged in LDS by DMA in two
    stages, so every K and V element a tile brings in serves 128 queries. A
    long key range is split over `splits` workgroups of `tilesPerSplit`
    tiles each; they write unnormalised partial records (o, running max m,
    sum l) that attention_f32_merge_kernel combines.

    Per wave and tile, S^T (64 keys x 32 queries) = K Q^T as two 32 x 32
    blocks of D/2 products, each over two dims: lanes 0-31 supply dim s and
    lanes 32-63 dim D/2 + s, so a lane's B operands are its query's half row,
    held in registers. Register r of a score block holds key
    8 (r / 4) + 4 (lane / 32) + r % 4 of the block for query lane % 32; that
    register is directly the B operand of one P.V product, O^T (D x 32) +=
    V^T P^T, whose A operand is then the V row of that key. The operand reads
    of both products run AH steps ahead of their MFMAs, and the two score
    blocks (and the D/32 output tiles) are independent accumulator chains.

    LDS K rows keep 16-byte block c at c ^ (row % 16), so the 16 rows one
    A-operand read touches hit distinct banks; V rows are natural.
*/
constexpr int TK = 64;     // keys per tile
constexpr int TQ = 128;    // query tokens per workgroup

/* s_waitcnt vmcnt(0), the other counters left alone */
__device__ __forceinline__ void wait_vmcnt_all() {
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
}

struct TileArgs {
    AttentionF32Params p;
    float* acc;              // split records [split][head][token][dim]
    float2* ml;              // their (m, l) [split][head][token]
    uint32_t groups;         // token groups of TQ
    uint32_t splits;         // workgroups per (token group, head)
    uint32_t tilesPerSplit;  // key tiles per workgroup when splits > 1
};

/* the key tiles of token group `grp`: every key a token of the group sees
   lies in [kbeg, kbeg + TK * ntiles) */
__host__ __device__ inline void group_tiles(uint64_t count, uint64_t start, uint64_t window, uint64_t grp,
                                            uint64_t& kbeg, uint32_t& ntiles) {
    const uint64_t t0 = grp * TQ;
    const uint64_t tLast = (t0 + TQ < count ? t0 + TQ : count) - 1;
    const uint64_t p0 = start + t0, p1 = start + tLast;
    const uint64_t first = window && p0 + 1 > window ? p0 + 1 - window : 0;
    kbeg = first / TK * TK;
    ntiles = uint32_t((p1 + 1 - kbeg + TK - 1) / TK);
}

template <int D>
__global__ __launch_bounds__(256) void attention_f32_tile_kernel(TileArgs a) {
    constexpr int DT = D / 32;             // 32-dim tiles of O^T
    constexpr int HALF = D / 2;            // q elements per lane
    constexpr int NI = HALF / 4;           // 16-byte q pieces per lane
    constexpr int CPR = D / 4;             // 16-byte blocks per row
    constexpr int TILE = TK * D;           // floats per K or V tile
    constexpr int BPW = TILE * 4 / 1024 / 4;   // 1 KB DMA blocks per wave per tile (K or V)
    constexpr int AH = 2;                  // operand reads in flight ahead of their products
    __shared__ __attribute__((aligned(16))) float Ks[2 * TILE];
    __shared__ __attribute__((aligned(16))) float Vs[2 * TILE];

    const AttentionF32Params& p = a.p;
    const int lane = threadIdx.x & 63, h = lane >> 5, j = lane & 31;
    const uint32_t w = __builtin_amdgcn_readfirstlane(uint32_t(threadIdx.x >> 6));
    uint32_t bid = blockIdx.x;
    const uint32_t sigma = bid % a.splits;
    bid /= a.splits;
    const uint64_t head = bid % uint32_t(p.heads);
    const uint64_t grp = a.groups - 1 - bid / uint32_t(p.heads);   // the longest groups first
    uint64_t kbeg;
    uint32_t ntiles;
    group_tiles(p.count, p.start, p.window, grp, kbeg, ntiles);
    const uint32_t tBegin = a.splits > 1 ? sigma * a.tilesPerSplit : 0u;
    if (tBegin >= ntiles) return;   // the whole workgroup: no split here
    const uint32_t tEnd = a.splits > 1 && tBegin + a.tilesPerSplit < ntiles ? tBegin + a.tilesPerSplit : ntiles;

    const uint64_t kv = head / (p.heads / p.kvHeads);
    const uint64_t lastKey = p.start + p.count - 1;
    const uint64_t tw0 = grp * TQ + 32 * w;
    const bool waveRows = tw0 < p.count;
    const uint64_t t = tw0 + j;
    const bool rowValid = t < p.count;
    const uint64_t P = p.start + t;
    const uint64_t first = p.window && P + 1 > p.window ? P + 1 - p.window : 0;
    // keys any row of the wave sees: [wFirst, wLast]
    const uint64_t wLast = p.start + (tw0 + 31 < p.count ? tw0 + 31 : p.count - 1);
    const uint64_t wFirst = p.window && p.start + tw0 + 1 > p.window ? p.start + tw0 + 1 - p.window : 0;

    float qh[HALF];
    {
        const float* qrow = static_cast<const float*>(p.q) + (t * p.heads + head) * p.qStride + HALF * h;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const floatx4 v = rowValid ? *reinterpret_cast<const floatx4*>(qrow + 4 * i) : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int e = 0; e < 4; ++e) qh[4 * i + e] = v[e];
        }
    }

    // DMA of the tile at key k0 into stage st: block n of this wave covers
    // 16-byte slots 64 (BPW w + n) + lane, row slot / CPR; K row r takes its
    // block (slot % CPR) ^ (r % 16) from memory. Rows past the last key
    // repeat it (their scores are masked and their P is 0).
    const char* kbase = reinterpret_cast<const char*>(static_cast<const float*>(p.keys) + kv * p.headStride);
    const char* vbase = reinterpret_cast<const char*>(static_cast<const float*>(p.values) + kv * p.headStride);
    const uint32_t ldsK = lds_address(Ks), ldsV = lds_address(Vs);
    const uint32_t rowBytes = uint32_t(p.posStride) * 4;
    auto issue = [&](uint64_t k0, uint32_t st) __attribute__((always_inline)) {
        const uint32_t lim = uint32_t(lastKey - k0 < TK - 1 ? lastKey - k0 : TK - 1);
        const char* kt = kbase + k0 * rowBytes;
        const char* vt = vbase + k0 * rowBytes;
#pragma unroll
        for (int n = 0; n < BPW; ++n) {
            const uint32_t blk = w * BPW + n;
            const uint32_t slot = blk * 64 + lane, r = slot / CPR, cp = slot % CPR;
            const uint32_t rowOff = (r < lim ? r : lim) * rowBytes;
            const uint32_t lds = __builtin_amdgcn_readfirstlane(st * TILE * 4 + blk * 1024);
            dma_block(kt, rowOff + 16 * (cp ^ (r & 15)), ldsK + lds);
            dma_block(vt, rowOff + 16 * cp, ldsV + lds);
        }
    };

    floatx16 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] = 0.0f;
    float m = -INFINITY, lsum = 0.0f;
    const float scale = 1.0f / sqrtf(float(D));

    issue(kbeg + uint64_t(tBegin) * TK, 0);
    for (uint32_t it = tBegin; it < tEnd; ++it) {
        const uint32_t st = (it - tBegin) & 1;
        const uint64_t k0 = kbeg + uint64_t(it) * TK;
        // tile `it` (and, the first time, q) has landed for every wave, and
        // every wave is done with the other stage
        wait_vmcnt_all();
        lds_barrier();
        if (it + 1 < tEnd) issue(k0 + TK, st ^ 1);
        if (!waveRows || k0 > wLast || k0 + TK - 1 < wFirst) continue;   // uniform over the wave
        const float* ks = Ks + st * TILE;
        const float* vs = Vs + st * TILE;

        // S^T: step i takes dims HALF h + 4 i .. + 3 of both key blocks, its
        // K operands read AH steps ahead into a ring; the two blocks' chains
        // alternate, and the scheduling groups pin that order
        floatx16 s[2];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) s[b][r] = 0.0f;
        {
            auto kfrag = [&](int i, int b) __attribute__((always_inline)) {
                const int c = NI * h + i;
                return *reinterpret_cast<const floatx4*>(ks + (32 * b + j) * D + 4 * (c ^ (j & 15)));
            };
            floatx4 f[AH + 1][2];
#pragma unroll
            for (int i = 0; i < AH; ++i)
#pragma unroll
                for (int b = 0; b < 2; ++b) f[i][b] = kfrag(i, b);
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                if (i + AH < NI)
#pragma unroll
                    for (int b = 0; b < 2; ++b) f[(i + AH) % (AH + 1)][b] = kfrag(i + AH, b);
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                    for (int b = 0; b < 2; ++b)
                        s[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(f[i % (AH + 1)][b][e], qh[4 * i + e], s[b], 0, 0, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * AH, 0);
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                if (i + AH < NI) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
            }
        }
        // keys of the tile this row sees: offsets [lo, hi] from k0
        const int64_t hi64 = int64_t(P) - int64_t(k0), lo64 = int64_t(first) - int64_t(k0);
        const int hi = rowValid ? int(hi64 < TK ? hi64 : TK) : -1;
        const int lo = int(lo64 > TK ? TK + 1 : (lo64 > 0 ? lo64 : 0));
        float mx = -INFINITY;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = 32 * b + 8 * (r >> 2) + 4 * h + (r & 3);
                s[b][r] = key >= lo && key <= hi ? s[b][r] * scale : -INFINITY;
                mx = fmaxf(mx, s[b][r]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 32, WAVE));
        const float mn = fmaxf(m, mx);
        float alpha = 1.0f, psum = 0.0f;
        if (mn == -INFINITY) {   // no key of this row so far
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 16; ++r) s[b][r] = 0.0f;
        } else {
            alpha = expf(m - mn);
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    s[b][r] = expf(s[b][r] - mn);
                    psum += s[b][r];
                }
        }
        psum += __shfl_xor(psum, 32, WAVE);
        lsum = lsum * alpha + psum;
        m = mn;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;

        // P.V: step n = (b, r) takes key row 32 b + 8 (r / 4) + 4 h + r % 4 of
        // every d tile (DT independent chains), its V operands AH steps ahead
        {
            auto vfrag = [&](int n, int dt) __attribute__((always_inline)) {
                const int b = n >> 4, r = n & 15;
                return vs[(32 * b + 8 * (r >> 2) + 4 * h + (r & 3)) * D + 32 * dt + j];
            };
            float f[AH + 1][DT];
#pragma unroll
            for (int n = 0; n < AH; ++n)
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) f[n][dt] = vfrag(n, dt);
#pragma unroll
            for (int n = 0; n < 32; ++n) {
                if (n + AH < 32)
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) f[(n + AH) % (AH + 1)][dt] = vfrag(n + AH, dt);
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(f[n % (AH + 1)][dt], s[n >> 4][n & 15], o[dt], 0, 0, 0);
            }
            // the reads of a step pair up into DT / 2 two-address reads
            __builtin_amdgcn_sched_group_barrier(0x100, AH * DT / 2, 0);
#pragma unroll
            for (int n = 0; n < 32; ++n) {
                if (n + AH < 32) __builtin_amdgcn_sched_group_barrier(0x100, DT / 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, DT, 0);
            }
        }
    }
    if (!rowValid) return;

    // O^T register r of d tile dt holds dim 32 dt + 8 (r / 4) + 4 (lane / 32) + r % 4
    if (a.splits == 1) {
        const float inv = 1.0f / lsum;
        float* dst = p.out + (t * p.heads + head) * D;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<floatx4*>(dst + 32 * dt + 8 * g + 4 * h) =
                    floatx4{o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv, o[dt][4 * g + 2] * inv, o[dt][4 * g + 3] * inv};
        return;
    }
    const size_t rec = (size_t(sigma) * p.heads + head) * p.count + t;
    float* dst = a.acc + rec * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g)
            *reinterpret_cast<floatx4*>(dst + 32 * dt + 8 * g + 4 * h) =
                floatx4{o[dt][4 * g], o[dt][4 * g + 1], o[dt][4 * g + 2], o[dt][4 * g + 3]};
    if (h == 0) a.ml[rec] = make_float2(m, lsum);
}

/* one wave per (token, head): out = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s
   over the splits that cover the token's group (a split in which the row
   saw no key has m = -inf and adds nothing); the records of up to MB splits
   are loaded together, one memory round trip per MB splits */
template <int D>
__global__ __launch_bounds__(256) void attention_f32_merge_kernel(TileArgs a) {
    constexpr int MB = 16, NE = D / 64;
    const AttentionF32Params& p = a.p;
    const int lane = threadIdx.x & 63;
    const uint64_t task = uint64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (task >= p.count * p.heads) return;
    const uint64_t t = task / p.heads, head = task % p.heads;
    uint64_t kbeg;
    uint32_t ntiles;
    group_tiles(p.count, p.start, p.window, t / TQ, kbeg, ntiles);
    const uint32_t n = (ntiles + a.tilesPerSplit - 1) / a.tilesPerSplit;
    float M = -INFINITY, L = 0.0f, acc[NE] = {};
    for (uint32_t s0 = 0; s0 < n; s0 += MB) {
        float2 ml[MB];
        float av[MB][NE];
#pragma unroll
        for (int u = 0; u < MB; ++u) {
            const bool ok = s0 + u < n;
            const size_t rec = ((size_t(s0) + u) * p.heads + head) * p.count + t;
            ml[u] = ok ? a.ml[rec] : make_float2(-INFINITY, 0.0f);
#pragma unroll
            for (int i = 0; i < NE; ++i) av[u][i] = ok ? a.acc[rec * D + lane + 64 * i] : 0.0f;
        }
        float bm = M;
#pragma unroll
        for (int u = 0; u < MB; ++u) bm = fmaxf(bm, ml[u].x);
        if (bm == -INFINITY) continue;
        const float sc = expf(M - bm);   // 0 while nothing is merged
        L *= sc;
#pragma unroll
        for (int i = 0; i < NE; ++i) acc[i] *= sc;
#pragma unroll
        for (int u = 0; u < MB; ++u) {
            if (ml[u].x == -INFINITY) continue;
            const float e = expf(ml[u].x - bm);
            L += ml[u].y * e;
#pragma unroll
            for (int i = 0; i < NE; ++i) acc[i] += e * av[u][i];
        }
        M = bm;
    }
    const float inv = 1.0f / L;
    float* dst = p.out + task * D;
#pragma unroll
    for (int i = 0; i < NE; ++i) dst[lane + 64 * i] = acc[i] * inv;
}

/* whether the tiled form takes this call: fp32 q and KV, dim 64 or 128,
   every row and the output on 16-byte boundaries, a tile's rows within a
   32-bit byte offset */
bool tile_eligible(const AttentionF32Params& p) {
    auto aligned = [](const void* x) { return (reinterpret_cast<uintptr_t>(x) & 15) == 0; };
    return p.qType == 0 && p.kvType == 0 && (p.dim == 64 || p.dim == 128) && aligned(p.q) && aligned(p.keys) &&
           aligned(p.values) && aligned(p.out) && p.qStride % 4 == 0 && p.posStride % 4 == 0 &&
           p.headStride % 4 == 0 && p.posStride < (uint64_t(1) << 22);
}

bool launch_tiled(const AttentionF32Params& p, hipStream_t stream) {
    Context& ctx = Context::instance();
    TileArgs a{};
    a.p = p;
    const uint64_t groups = (p.count + TQ - 1) / TQ;
    uint64_t total = 0;
    uint32_t maxTiles = 0;
    for (uint64_t g = 0; g < groups; ++g) {
        uint64_t kbeg;
        uint32_t nt;
        group_tiles(p.count, p.start, p.window, g, kbeg, nt);
        total += nt;
        maxTiles = nt > maxTiles ? nt : maxTiles;
    }
    total *= p.heads;
    // split the key ranges when the (group, head) pairs alone leave workgroup
    // slots of the 256 CUs empty (one workgroup per CU at dim 128, two at 64),
    // and the records stay under 256 MB
    const uint64_t slots = p.dim == 64 ? 512 : 256;
    uint64_t tps = (total + slots - 1) / slots;
    const uint64_t perSplit = p.heads * p.count * (p.dim * 4 + 8);
    while (tps < maxTiles && ((maxTiles + tps - 1) / tps) * perSplit > (uint64_t(256) << 20)) tps *= 2;
    a.groups = uint32_t(groups);
    a.splits = tps < maxTiles ? uint32_t((maxTiles + tps - 1) / tps) : 1u;
    a.tilesPerSplit = a.splits > 1 ? uint32_t(tps) : maxTiles;
    const uint64_t blocks = groups * p.heads * a.splits;
    if (blocks > 0x7FFFFFFFull) return ctx.fail("attention: too many tasks");
    if (a.splits > 1) {
        const size_t accBytes = size_t(a.splits) * p.heads * p.count * p.dim * 4;
        char* parts = static_cast<char*>(ctx.grow(SLOT_ATTN_PARTS, size_t(a.splits) * perSplit));
        if (!parts) return false;
        a.acc = reinterpret_cast<float*>(parts);
        a.ml = reinterpret_cast<float2*>(parts + accBytes);
    }
    const bool d64 = p.dim == 64;
    if (!ctx.launch("attention_f32_tile_kernel", stream, [&] {
            if (d64) hipLaunchKernelGGL(attention_f32_tile_kernel<64>, dim3(unsigned(blocks)), dim3(256), 0, stream, a);
            else hipLaunchKernelGGL(attention_f32_tile_kernel<128>, dim3(unsigned(blocks)), dim3(256), 0, stream, a);
        }))
        return false;
    if (a.splits == 1) return true;
    const uint64_t mblocks = (p.count * p.heads + 3) / 4;
    return ctx.launch("attention_f32_merge_kernel", stream, [&] {
        if (d64) hipLaunchKernelGGL(attention_f32_merge_kernel<64>, dim3(unsigned(mblocks)), dim3(256), 0, stream, a);
        else hipLaunchKernelGGL(attention_f32_merge_kernel<128>, dim3(unsigned(mblocks)), dim3(256), 0, stream, a);
    });
}

} // namespace

bool launch_attention_f32(const AttentionF32Params& p, hipStream_t stream) {
    Context& ctx = Context::instance();
    if (p.dim == 0 || p.dim > MAX_DIM) return ctx.fail("attention: dim must be 1..256");
    if (p.kvHeads == 0 || p.heads % p.kvHeads) return ctx.fail("attention: heads must be a multiple of kvHeads");
    if (p.qStride < p.dim) return ctx.fail("attention: qStride < dim");
    const uint64_t tasks = p.count * p.heads;
    if (tasks == 0) return true;
    if (tile_eligible(p)) return launch_tiled(p, stream);
    const uint64_t blocks = (tasks + 3) / 4;
    if (blocks > 0x7FFFFFFFull) return ctx.fail("attention: too many tasks");
    return ctx.launch("attention_f32_kernel", stream, [&] {
        hipLaunchKernelGGL(attention_f32_kernel, dim3(unsigned(blocks)), dim3(256), 0, stream, p);
    });
}

} // namespace aigpu
