// qlinear.hip -- the C-ABI of the fused IQR-linear + LoRA forward and backward (include/r97q.h):
// argument checks, workspace layout and the launch order of the stages.
//
//   forward   t = X.A^T; Y = X.W^T + s.t.B^T          (reference twins: src/adjoint/host/linear.cpp:
//                                                      193-219, lora.cpp:226-244, 416-441)
//   backward  dt = s.dY.B;  dX = dY.W + dt.A;          (linear.cpp:221-243, lora.cpp:260-328,
//             dA += dt^T.X;  dB += s.dY^T.t            451-521)
//
// Kernels: the fused decode + MFMA base products (qlinear_rt.hip, fed the token operand from
// its tiled copy in the workspace) carry the adapter's up-projection in their epilogue; the
// adapter's down products, factor gradients and the token operand's tiled copy are lora.hip's; in
// the fused backward the gradient launch leaves its chunk sums for the dX launch to add (the
// stand-alone gradient entry adds them in its own launch).
// The coded trunk's dX (the activation's group scale in the epilogue) and the vocabulary head run
// the LDS-staged kernels of qlinear_fused.hip on the row-major operand.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>

#include "act_tiles.h"
#include "iqr_device.h"
#include "lora.h"
#include "qlinear_fused.h"
#include "qlinear_q.h"
#include "qlinear_rt.h"
#include "status.h"

#include <atomic>

using namespace r97q;

namespace {

int64_t align256(int64_t b) { return (b + 255) & ~(int64_t)255; }

bool rank_ok(int r) { return r == 0 || r == 8 || r == 16 || r == 32 || r == 64; }

// One call's shape. `once` is the decode-once choice, read once when the entry builds its shape:
// every workspace layout and launch of that call follows the same choice, whatever another
// thread sets meanwhile.
struct Shape {
    int64_t T, N, K;
    int r;
    bool once;
};

// The base products either decode each weight tile in the main loop, once for every 512-token
// panel (the fused kernel), or decode the whole weight once a call into the workspace and run the
// product over the decoded tiles (rt::launch_predecode, then rt::launch_pd). The second saves the
// repeated decode's VALU work and power, but costs a launch that writes and re-reads N*K*2 bytes.
// Measured on the card (one whole LoRA step each):
//   - it loses at 8 panels (C2's 4096 tokens: 328 us a step against 313);
//   - at 16 panels (8192 tokens) it wins for weights of 8M values and more (4096 x 4096: 0.64 ms
//     against 0.70; C3's MLP block: 4.99 ms against 5.11; a C5 layer: 2.02 against 2.13) and loses
//     for 2048 x 2048 (0.229 ms against 0.214);
//   - it wins at 32 and 64 panels (4096 x 4096 at 16384 tokens: 1.21 ms against 1.27; C5's 32768
//     tokens: the 24-layer step 182 ms against 191).
// r97q_set_decode_once overrides the choice; the entry that allocates nothing always runs the
// fused kernel.
constexpr int64_t kDecodeOnceMinT = 32 * rt::kBM;          // any weight from 16384 tokens
constexpr int64_t kDecodeOnceMinTLarge = 16 * rt::kBM;     // weights of kDecodeOnceLarge values from 8192
constexpr int64_t kDecodeOnceLarge = int64_t(1) << 23;
std::atomic<int> g_decode_once{R97Q_DECODE_AUTO};
Shape shape(int64_t T, int64_t N, int64_t K, int r) {
    const int m = g_decode_once.load(std::memory_order_relaxed);
    const bool once = m != R97Q_DECODE_AUTO ? m == R97Q_DECODE_ONCE
                                            : T >= kDecodeOnceMinT || (T >= kDecodeOnceMinTLarge && N * K >= kDecodeOnceLarge);
    return Shape{T, N, K, r, once};
}

// Split-K of the fused kernel (rt::Params::ksplit, nfull). A launch holds tiles = ceil(T/512) x
// outputs/128 workgroups, one a CU at a time over the card's 256 CUs. When the tiles leave much of
// the last round of CUs idle and the reduction is long, the reductions of the tiles past nfull are
// dealt over S ranges each (a workgroup a range), each range's f32 partial product written to the
// workspace and added in range order by a second launch. Two forms: every tile split (nfull 0: a
// launch of fewer tiles than CUs), or the whole rounds' tiles run whole and only the tiles of the
// partial last round split (nfull = 256 x whole rounds), so the last round runs on every CU for
// 1/S of a tile's time and only its tiles write partials. The choice minimises a model of the
// launch's time in microseconds, measured at C2 and at the reference's published shapes: a 64-deep
// step of a full round of tiles takes ~1.85 us, a partial last round with a fraction f of the CUs
// busy runs at a higher clock and takes (0.4 + 0.6 f) of a full round's time, a round's prologue
// and epilogue ~3 us, and the partials cost their bytes written and read (S x split tiles x
// 512 x 128 x 8; the writes overlap other workgroups' products) at ~10 TB/s plus ~4 us for the
// added launch. A split needs at least 16 steps a range and must beat no split by 7%.
// Deterministic in the shape, so a call's bits never depend on anything else.
constexpr int kSplitMax = 8;
struct Split {
    int S;      // ranges a split tile's reduction is dealt over (1: no split)
    int nfull;  // tiles run whole, before the split ones (every tile when S is 1)
};
Split split_for(int64_t T, int64_t outputs, int64_t red) {
    const int64_t tiles = ((T + rt::kBM - 1) / rt::kBM) * (outputs / rt::kBN);
    const int64_t nsteps = red / rt::kStep;
    auto rounds = [](double u) {
        const double full = std::floor(u), frac = u - full;
        return full + (frac > 0 ? 0.4 + 0.6 * frac : 0.0);
    };
    auto cost = [&](int64_t nfull, int S) {
        double t = rounds((double)nfull / 256.0) * ((double)nsteps * 1.85 + 3.0);
        if (S > 1) {
            const int64_t rest = tiles - nfull;
            t += rounds((double)(rest * S) / 256.0) * ((double)nsteps / S * 1.85 + 3.0);
            t += (double)S * (double)rest * rt::kBM * rt::kBN * 8.0 / 1.0e7 + 4.0;
        }
        return t;
    };
    const double t1 = cost(tiles, 1);
    Split best{1, (int)tiles};
    double best_t = t1;
    const int64_t whole = tiles / 256 * 256;  // the whole rounds' tiles
    for (int64_t nfull : {(int64_t)0, whole}) {
        if (nfull > 0 && nfull == tiles) continue;
        for (int S = 2; S <= kSplitMax; ++S) {
            if (nsteps / S < 16) break;
            const double t = cost(nfull, S);
            if (t < 0.93 * t1 && t < best_t) {
                best = Split{S, (int)nfull};
                best_t = t;
            }
        }
    }
    return best;
}

// Workspace layout. Forward: Xt (X's tiled copy, act_tiles.h) | P [T, 2r] | Apad [rd, K] (when r
// is not a multiple of 16) | Wt (the weight's decoded tiles, rt::wt_bytes, when decode_once).
// Backward: dYt (dY's tiled copy) | At [K, r] | P [T, 2r] | PtA [2r, ldt] | PtB [2r, ldt]
// | partA [chunks, r, K] | partB [chunks, r, N] (f32 partial sums of the factor gradients) | done
// (bwd_counters) | Wt (as the forward's).
// Either direction then holds Sp [S, split tiles, 512, 128] f32: the split-K partials, when the fused
// kernel splits (ksplit > 1; never on the decode-once path, nor for the entry that allocates
// nothing).
// Wt and Sp are -1 where the layout has none.
struct FwdWs {
    int64_t Xt, P, Apad, Wt, Sp, total;
    int ksplit, nfull;
};
FwdWs fwd_ws(const Shape& s, bool fused_only = false) {
    FwdWs w{};
    w.Xt = 0;
    w.P = w.Xt + align256(act_tile_bytes(s.T, s.K));
    w.total = w.P;
    if (s.r > 0) {
        const int rd = down_rank(s.r);
        w.Apad = w.P + align256(s.T * 2 * s.r * 2);
        w.total = w.Apad + (rd != s.r ? align256((int64_t)rd * s.K * 2) : 0);
    }
    w.Wt = w.Sp = -1;
    w.ksplit = 1;
    if (!fused_only && s.once) {
        w.Wt = w.total;
        w.total += align256(rt::wt_bytes(s.N, s.K));
    } else if (!fused_only) {
        const Split sp = split_for(s.T, s.N, s.K);
        w.ksplit = sp.S;
        w.nfull = sp.nfull;
        if (w.ksplit > 1) {
            w.Sp = w.total;
            w.total += align256(rt::split_bytes(sp.S, ((s.T + rt::kBM - 1) / rt::kBM) * (s.N / rt::kBN) - sp.nfull));
        }
    }
    return w;
}
struct BwdWs {
    int64_t dYt, At, P, PtA, PtB, partA, partB, done, Wt, Sp, total;
    int ksplit, nfull;
};
// the backward's counters, zeroed by its down product: the gradient launch's column blocks (dA's,
// then dB's)
int64_t bwd_counters(const Shape& s) { return grad_blocks(s.K) + grad_blocks(s.N); }
void bwd_ws_wt(const Shape& s, BwdWs& w) {
    w.Wt = w.Sp = -1;
    w.ksplit = 1;
    if (s.once) {
        w.Wt = w.total;
        w.total += align256(rt::wt_bytes(s.N, s.K));
    } else {
        const Split sp = split_for(s.T, s.K, s.N);
        w.ksplit = sp.S;
        w.nfull = sp.nfull;
        if (w.ksplit > 1) {
            w.Sp = w.total;
            w.total += align256(rt::split_bytes(sp.S, ((s.T + rt::kBM - 1) / rt::kBM) * (s.K / rt::kBN) - sp.nfull));
        }
    }
}
BwdWs bwd_ws(const Shape& s) {
    BwdWs w{};
    w.dYt = 0;
    w.At = w.dYt + align256(act_tile_bytes(s.T, s.N));
    if (s.r == 0) {
        w.total = w.At;
        bwd_ws_wt(s, w);
        return w;
    }
    const int64_t ldt = grad_ld(s.T);
    w.P = w.At + align256(s.K * s.r * 2);
    w.PtA = w.P + align256(s.T * 2 * s.r * 2);
    w.PtB = w.PtA + align256(2 * s.r * ldt * 2);
    // the chunk partials of either factor's gradient: as many as its launch alone takes (the most)
    const int64_t chunksA = grad_chunks(s.T, s.K, 0);
    const int64_t chunksB = grad_chunks(s.T, 0, s.N);
    w.partA = w.PtB + align256(2 * s.r * ldt * 2);
    w.partB = w.partA + align256(chunksA * s.r * s.K * 4);
    w.done = w.partB + align256(chunksB * s.r * s.N * 4);
    w.total = w.done + align256(bwd_counters(s) * 4);
    bwd_ws_wt(s, w);
    return w;
}

// The adapter rows on their own (the shrink's and the expand's adjoints), workspace layouts:
// shrink: P [T, 2r] | Pt [2r, ldt] | At [K, r] | part [chunks, r, K] | done
// expand: Bt [rd, N] | Pt2 [2r, ldt] | part [chunks, r, N] | done
struct ShrinkWs {
    int64_t P, Pt, At, part, done, total;
};
ShrinkWs shrink_ws(int64_t T, int64_t K, int r) {
    ShrinkWs w{};
    if (r == 0) return w;
    const int64_t ldt = grad_ld(T);
    w.P = 0;
    w.Pt = w.P + align256(T * 2 * r * 2);
    w.At = w.Pt + align256(2 * r * ldt * 2);
    w.part = w.At + align256(K * r * 2);
    w.done = w.part + align256(grad_chunks(T, K, 0) * r * K * 4);
    w.total = w.done + align256(grad_blocks(K) * 4);
    return w;
}
struct ExpandWs {
    int64_t Bt, Pt2, part, done, total;
};
ExpandWs expand_ws(int64_t T, int64_t N, int r) {
    ExpandWs w{};
    if (r == 0) return w;
    const int64_t ldt = grad_ld(T);
    w.Bt = 0;
    w.Pt2 = w.Bt + align256((int64_t)down_rank(r) * N * 2);
    w.part = w.Pt2 + align256(2 * r * ldt * 2);
    w.done = w.part + align256(grad_chunks(T, 0, N) * r * N * 4);
    w.total = w.done + align256(grad_blocks(N) * 4);
    return w;
}

// The coded shrink's adjoint: P [T, 2r] | Pt [2r, ldt] | At [K, r] | g [T, K] f32 | xhi, xlo [T, K]
// bf16 | part [chunks, r, K] f32 | done.
struct ShrinkQWs {
    int64_t P, Pt, At, g, xhi, xlo, part, done, total;
};
ShrinkQWs shrink_q_ws(int64_t T, int64_t K, int r) {
    ShrinkQWs w{};
    if (r == 0) return w;
    const int64_t ldt = grad_ld(T);
    w.P = 0;
    w.Pt = w.P + align256(T * 2 * r * 2);
    w.At = w.Pt + align256(2 * r * ldt * 2);
    w.g = w.At + align256(K * r * 2);
    w.xhi = w.g + align256(T * K * 4);
    w.xlo = w.xhi + align256(T * K * 2);
    w.part = w.xlo + align256(T * K * 2);
    w.done = w.part + align256(grad_chunks(T, K, 0) * r * K * 4);
    w.total = w.done + align256(grad_blocks(K) * 4);
    return w;
}

// the width of one activation-scale group over k columns, read back from `groups` scale columns
// (src/adjoint/host/lora.cpp:70-77): the power of two whose ceiling division gives `groups`, else
// ceil(k / groups); one group spans the row
int64_t group_width(int64_t k, int64_t groups) {
    if (k <= 0) return 1;
    if (groups <= 1) return k;
    const int64_t lo = (k + groups - 1) / groups;
    int64_t b = 1;
    while (b < lo) b <<= 1;
    return (k + b - 1) / b == groups ? b : lo;
}

// zero-fill + copy of a [r, cols] bf16 matrix into [rd, cols] (rows r..rd-1 zero)
__global__ __launch_bounds__(256) void pad_rows16(const uint16_t* __restrict__ in, int r, int rd,
                                                  int64_t cols, uint16_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)rd * cols) return;
    const int64_t row = i / cols;
    out[i] = row < r ? in[i] : (uint16_t)0;
}

int check_weight(const R97qWeight* w) {
    if (!w || !w->stream || !w->scale_t) {
        set_error("qlinear: null weight");
        return R97Q_EINVAL;
    }
    const bool codes8 = w->bits == R97Q_CODES8;
    if (!codes8 && (!w->mad || w->state_bits != 16 || w->bits < 3 || w->bits > 6)) {
        set_error("qlinear: weight form not served (trellis.mad, L 16, bits 3..6, or the int8-code form)");
        return R97Q_EUNSUPPORTED;
    }
    if (w->rows % kBN != 0 || w->cols % kBN != 0 || (!codes8 && w->run_rows % 32 != 0)) {
        set_error("qlinear: N %lld and K %lld must be multiples of 128, run %d of 32",
                  (long long)w->rows, (long long)w->cols, (int)w->run_rows);
        return R97Q_EUNSUPPORTED;
    }
    return R97Q_OK;
}

}  // namespace

// ---------------------------------------------------------------- the stages
namespace {

int check_rank(int32_t rank, const char* who) {
    if (!rank_ok(rank)) {
        set_error("%s: rank %d not served (0, 8, 16, 32, 64)", who, (int)rank);
        return R97Q_EUNSUPPORTED;
    }
    return R97Q_OK;
}

int check_ws(int64_t have, int64_t need, const void* ws, const char* who) {
    if (have < need || (need > 0 && !ws)) {
        set_error("%s: workspace %lld bytes, needs %lld", who, (long long)have, (long long)need);
        return R97Q_EWORKSPACE;
    }
    return R97Q_OK;
}

// t = X.A^T (f32, kept for the backward), P = [hi | lo](s.t) in the forward workspace
int fwd_prep(const Shape& sh, const uint16_t* X, const uint16_t* A, float scale, float* t_out,
             uint8_t* wsb, hipStream_t s) {
    const FwdWs ws = fwd_ws(sh);
    uint16_t* Xt = reinterpret_cast<uint16_t*>(wsb + ws.Xt);
    // rank 0: the tiled copy alone; else the down product writes it as it reads X
    if (sh.r == 0) return launch_act_tile(X, sh.T, sh.K, Xt, s);
    const int rank = sh.r, rd = down_rank(rank);
    const uint16_t* Wd = A;
    if (rd != rank) {
        uint16_t* Apad = reinterpret_cast<uint16_t*>(wsb + ws.Apad);
        hipLaunchKernelGGL(pad_rows16, dim3((unsigned)((rd * sh.K + 255) / 256)), dim3(256), 0, s, A,
                           rank, rd, sh.K, Apad);
        if (int e = launch_status("pad_rows16")) return e;
        Wd = Apad;
    }
    DownArgs a{};
    a.In = X;
    a.W = Wd;
    a.T = sh.T;
    a.Kin = sh.K;
    a.ldt = sh.T;
    a.r = rank;
    a.sa = 1.0f;
    a.sb = scale;
    a.out = t_out;
    a.P = reinterpret_cast<uint16_t*>(wsb + ws.P);
    a.tiled = Xt;
    return launch_lora_down(a, s);
}

// the register-fed product over the token operand's tiled copy `act` (forward or dX): with `wt`
// (rt::wt_bytes of workspace) the weight decoded once into it, then the product over its tiles;
// without, the fused kernel decoding in its main loop
int rt_base(const R97qWeight* w, bool fwd, const Shape& sh, const uint16_t* act, const uint16_t* P,
            const uint16_t* Q, void* out, int32_t out_dtype, int32_t accumulate, uint8_t* wt, hipStream_t s,
            const rt::Params::Sums* sums = nullptr, int ksplit = 1, int nfull = 0, float* part = nullptr) {
    rt::Params p{};
    p.act = act;
    p.T = sh.T;
    p.N = sh.N;
    p.K = sh.K;
    p.stream = w->stream;
    p.scale_t = w->scale_t;
    p.a24 = w->mad_a & 0xFFFFFFu;
    p.b = w->mad_b;
    p.run_rows = w->run_rows;
    p.P = sh.r > 0 ? P : nullptr;
    p.Q = sh.r > 0 ? Q : nullptr;
    p.rank = sh.r;
    p.out = out;
    p.out_f32 = out_dtype == R97Q_F32;
    p.accumulate = accumulate != 0;
    p.mtiles = (int)((sh.T + rt::kBM - 1) / rt::kBM);
    p.otiles = (int)((fwd ? sh.N : sh.K) / rt::kBN);
    p.wt = wt;
    p.ksplit = wt || !part ? 1 : ksplit;
    p.nfull = p.ksplit > 1 ? nfull : p.mtiles * p.otiles;
    p.part = p.ksplit > 1 ? part : nullptr;
    if (sums && !fwd) {
        p.sums[0] = sums[0];
        p.sums[1] = sums[1];
    }
    if (wt) {
        switch (w->bits) {
            case 3: rt::launch_predecode<3>(p, fwd, wt, s); break;
            case 4: rt::launch_predecode<4>(p, fwd, wt, s); break;
            case 5: rt::launch_predecode<5>(p, fwd, wt, s); break;
            case 6: rt::launch_predecode<6>(p, fwd, wt, s); break;
            default: rt::launch_predecode<R97Q_CODES8>(p, fwd, wt, s); break;
        }
        if (int e = launch_status("predecode_kernel")) return e;
        rt::launch_pd(p, fwd, s);
        return launch_status(fwd ? "qlinear_pd_kernel<fwd>" : "qlinear_pd_kernel<dx>");
    }
    auto go = [&](auto fwd_fn, auto dx_fn) { fwd ? fwd_fn(p, s) : dx_fn(p, s); };
    switch (w->bits) {
        case 3: go(rt::launch_fwd<3>, rt::launch_dx<3>); break;
        case 4: go(rt::launch_fwd<4>, rt::launch_dx<4>); break;
        case 5: go(rt::launch_fwd<5>, rt::launch_dx<5>); break;
        case 6: go(rt::launch_fwd<6>, rt::launch_dx<6>); break;
        default: go(rt::launch_fwd<R97Q_CODES8>, rt::launch_dx<R97Q_CODES8>); break;
    }
    if (int e = launch_status(fwd ? "qlinear_rt_kernel<fwd>" : "qlinear_rt_kernel<dx>")) return e;
    if (p.ksplit > 1) {
        rt::launch_split_reduce(p, fwd, s);
        return launch_status("split_reduce_kernel");
    }
    return R97Q_OK;
}

int fwd_base(const R97qWeight* w, const Shape& sh, const uint16_t* B, void* Y, int32_t y_dtype, uint8_t* wsb,
             hipStream_t s, bool fused_only = false) {
    const FwdWs ws = fwd_ws(sh, fused_only);
    return rt_base(w, true, sh, reinterpret_cast<const uint16_t*>(wsb + ws.Xt),
                   reinterpret_cast<const uint16_t*>(wsb + ws.P), B, Y, y_dtype, 0,
                   ws.Wt >= 0 ? wsb + ws.Wt : nullptr, s, nullptr, ws.ksplit, ws.nfull,
                   ws.Sp >= 0 ? reinterpret_cast<float*>(wsb + ws.Sp) : nullptr);
}

// B^T [rd, N] (zero rows past r), A^T [K, r]; dt = s.dY.B as P = [hi | lo](dt) for the fused dX
// epilogue and PtA (the same, transposed) for dA; PtB = [hi | lo](s.t) transposed for dB.
int bwd_prep(const Shape& sh, const uint16_t* dY, const uint16_t* A, const uint16_t* B, const float* t,
             float scale, uint8_t* wsb, hipStream_t s) {
    const BwdWs ws = bwd_ws(sh);
    uint16_t* dYt = reinterpret_cast<uint16_t*>(wsb + ws.dYt);
    if (sh.r == 0) return launch_act_tile(dY, sh.T, sh.N, dYt, s);
    DownArgs a{};
    a.In = dY;
    a.W = B;
    a.w_kmajor = 1;
    a.tr_in = A;
    a.tr_out = reinterpret_cast<uint16_t*>(wsb + ws.At);
    a.tr_cols = sh.K;
    a.T = sh.T;
    a.Kin = sh.N;
    a.ldt = grad_ld(sh.T);
    a.r = sh.r;
    a.sa = scale;
    a.sb = scale;
    a.P = reinterpret_cast<uint16_t*>(wsb + ws.P);
    a.Pt = reinterpret_cast<uint16_t*>(wsb + ws.PtA);
    a.tiled = dYt;
    a.zero = reinterpret_cast<int*>(wsb + ws.done);
    a.nzero = (int)bwd_counters(sh);
    if (t) {
        a.U2 = t;
        a.s2 = scale;
        a.Pt2 = reinterpret_cast<uint16_t*>(wsb + ws.PtB);
    }
    return launch_lora_down(a, s);
}

// the token chunks of the gradient launch for the factor gradients asked for
int64_t grad_launch_chunks(const Shape& sh, bool dA, bool dB) {
    const int64_t chunk = grad_chunk_rows(sh.T, dA ? sh.K : 0, dB ? sh.N : 0);
    return (grad_ld(sh.T) + chunk - 1) / chunk;
}

// dA[j][k] += sum_m dt[m][j] X[m][k];  dB[n][j] += s . sum_m dY[m][n] t[m][j]. With `defer` the
// launch leaves its chunk sums in partA / partB for the dX launch to add (dx_base's dA, dB).
int bwd_grads(const Shape& sh, const uint16_t* X, const uint16_t* dY, float* dA, float* dB, uint8_t* wsb,
              hipStream_t s, bool defer = false) {
    const BwdWs ws = bwd_ws(sh);
    GradArgs g{};
    g.T = sh.T;
    g.ldt = grad_ld(sh.T);
    g.chunk = grad_chunk_rows(sh.T, dA ? sh.K : 0, dB ? sh.N : 0);
    g.defer = defer;
    int nz = 0;
    int* done = reinterpret_cast<int*>(wsb + ws.done);
    if (dA)
        g.one[nz++] = GradOne{reinterpret_cast<const uint16_t*>(wsb + ws.PtA), X, sh.K, dA, 1.0f, 0,
                              reinterpret_cast<float*>(wsb + ws.partA), done};
    if (dB)
        g.one[nz++] = GradOne{reinterpret_cast<const uint16_t*>(wsb + ws.PtB), dY, sh.N, dB, 1.0f, 1,
                              reinterpret_cast<float*>(wsb + ws.partB), done + grad_blocks(sh.K)};
    if (nz == 0) return R97Q_OK;
    return launch_lora_grads(sh.r, g, nz, s);
}

// dX; with dA / dB (rank > 0, after a deferred bwd_grads for the same factors) the same launch
// then adds the gradient launch's chunk sums into them
int dx_base(const R97qWeight* w, const Shape& sh, void* dX, int32_t dx_dtype, int32_t accumulate, uint8_t* wsb,
            hipStream_t s, float* dA = nullptr, float* dB = nullptr) {
    const BwdWs ws = bwd_ws(sh);
    rt::Params::Sums sums[2] = {};
    if (sh.r > 0 && (dA || dB)) {
        const int chunks = (int)grad_launch_chunks(sh, dA != nullptr, dB != nullptr);
        if (dA) sums[0] = {reinterpret_cast<const float*>(wsb + ws.partA), sh.K, chunks, 0, dA};
        if (dB) sums[1] = {reinterpret_cast<const float*>(wsb + ws.partB), sh.N, chunks, 1, dB};
    }
    return rt_base(w, false, sh, reinterpret_cast<const uint16_t*>(wsb + ws.dYt),
                   reinterpret_cast<const uint16_t*>(wsb + ws.P), reinterpret_cast<const uint16_t*>(wsb + ws.At), dX,
                   dx_dtype, accumulate, ws.Wt >= 0 ? wsb + ws.Wt : nullptr, s,
                   sums[0].part || sums[1].part ? sums : nullptr, ws.ksplit, ws.nfull,
                   ws.Sp >= 0 ? reinterpret_cast<float*>(wsb + ws.Sp) : nullptr);
}

// the LDS-staged dX kernel over row-major dY with the coded trunk's activation scale in its
// epilogue (no adapter, no workspace)
int dx_scaled(const R97qWeight* w, const Shape& sh, const uint16_t* dY, void* dX, int32_t dx_dtype,
              int32_t accumulate, hipStream_t s, const float* a_scale) {
    DxParams p{};
    p.a_scale = a_scale;
    p.a_scale_ld = sh.K / kBN;
    p.dY = dY;
    p.T = sh.T;
    p.N = sh.N;
    p.K = sh.K;
    p.stream = w->stream;
    p.scale_t = w->scale_t;
    p.a24 = w->mad_a & 0xFFFFFFu;
    p.b = w->mad_b;
    p.run_rows = w->run_rows;
    p.P = nullptr;
    p.At = nullptr;
    p.rank = 0;
    p.dX = dX;
    p.dx_f32 = dx_dtype == R97Q_F32;
    p.accumulate = accumulate != 0;
    p.mtiles = (int)((sh.T + kBM - 1) / kBM);
    p.ktiles = (int)(sh.K / kBN);
    switch (w->bits) {
        case 3: launch_dx<3>(p, s); break;
        case 4: launch_dx<4>(p, s); break;
        case 5: launch_dx<5>(p, s); break;
        case 6: launch_dx<6>(p, s); break;
        default: launch_dx<R97Q_CODES8>(p, s); break;
    }
    return launch_status("qlinear_dx_kernel");
}

int shape_ok(int64_t T, int64_t N, int64_t K, const char* who) {
    if (T <= 0 || N <= 0 || K <= 0 || N % kBN || K % kBN) {
        set_error("%s: T %lld N %lld K %lld (T > 0, N and K multiples of 128)", who, (long long)T,
                  (long long)N, (long long)K);
        return R97Q_EINVAL;
    }
    return R97Q_OK;
}

}  // namespace

// ---------------------------------------------------------------- the forward with no allocation
// The forward's workspace (the token operand's tiled copy, the adapter's [hi | lo] splits) held in a
// file-scope device array instead of a caller's buffer, for callers that cannot allocate. Each GPU
// holds its own copy of the array; host code reaches it only through the address
// hipGetSymbolAddress gives on that device (the array's name is a host-side stand-in there). Calls
// that overlap on one GPU share it and race; nothing in it needs to start at zero (the forward
// writes every byte it reads).
constexpr int64_t kNoAllocScratchBytes = int64_t(48) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kNoAllocDevices = 64;
void* g_scratch_at[kNoAllocDevices] = {};

// this device's scratch address, looked up once per device with that device current
int scratch_of_current_device(uint8_t** at, const char* who) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kNoAllocDevices) {
        set_error("%s: no current device (or device %d past %d)", who, dev, kNoAllocDevices);
        return R97Q_ELAUNCH;
    }
    void* p = __atomic_load_n(&g_scratch_at[dev], __ATOMIC_ACQUIRE);
    if (p == nullptr) {
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            set_error("%s: hipGetSymbolAddress(scratch) on device %d: %s", who, dev, hipGetErrorString(e));
            return R97Q_ELAUNCH;
        }
        __atomic_store_n(&g_scratch_at[dev], p, __ATOMIC_RELEASE);
    }
    *at = static_cast<uint8_t*>(p);
    return R97Q_OK;
}
}  // namespace

extern "C" {

int32_t r97q_set_decode_once(int32_t mode) {
    if (mode != R97Q_DECODE_AUTO && mode != R97Q_DECODE_ONCE && mode != R97Q_DECODE_FUSED) return -1;
    return g_decode_once.exchange(mode);
}

int64_t r97q_fwd_workspace_bytes(int64_t T, int64_t N, int64_t K, int32_t rank) {
    return fwd_ws(shape(T, N, K, rank)).total;
}

int64_t r97q_bwd_workspace_bytes(int64_t T, int64_t N, int64_t K, int32_t rank) {
    return bwd_ws(shape(T, N, K, rank)).total;
}

int r97q_lora_fwd_prep(int64_t T, int64_t N, int64_t K, const uint16_t* X, const uint16_t* A,
                       int32_t rank, float scale, float* t_out, void* workspace,
                       int64_t workspace_bytes, R97IqrStream stream) {
    clear_error();
    const char* who = "r97q_lora_fwd_prep";
    if (int e = shape_ok(T, N, K, who)) return e;
    if (int e = check_rank(rank, who)) return e;
    if (!X || (rank > 0 && (!A || !t_out))) {
        set_error("%s: null X, or A or t_out with rank > 0", who);
        return R97Q_EINVAL;
    }
    const Shape sh = shape(T, N, K, rank);
    if (int e = check_ws(workspace_bytes, fwd_ws(sh).total, workspace, who)) return e;
    return fwd_prep(sh, X, A, scale, t_out, static_cast<uint8_t*>(workspace), (hipStream_t)stream);
}

int r97q_qlinear_fwd_base(const R97qWeight* w, const uint16_t* X, int64_t T, const uint16_t* B,
                          int32_t rank, void* Y, int32_t y_dtype, void* workspace,
                          int64_t workspace_bytes, R97IqrStream stream) {
    clear_error();
    const char* who = "r97q_qlinear_fwd_base";
    if (int e = check_weight(w)) return e;
    if (int e = check_rank(rank, who)) return e;
    if (!X || !Y || T <= 0 || (rank > 0 && !B)) {
        set_error("%s: null X / Y (or B with rank > 0), or T <= 0", who);
        return R97Q_EINVAL;
    }
    const Shape sh = shape(T, w->rows, w->cols, rank);
    if (int e = check_ws(workspace_bytes, fwd_ws(sh).total, workspace, who)) return e;
    return fwd_base(w, sh, B, Y, y_dtype, static_cast<uint8_t*>(workspace), (hipStream_t)stream);
}

int r97q_qlinear_lora_fwd(const R97qWeight* w, const uint16_t* X, int64_t T, const uint16_t* A,
                          const uint16_t* B, int32_t rank, float scale, void* Y, int32_t y_dtype,
                          float* t_out, void* workspace, int64_t workspace_bytes,
                          R97IqrStream stream) {
    clear_error();
    const char* who = "r97q_qlinear_lora_fwd";
    if (int e = check_weight(w)) return e;
    if (int e = check_rank(rank, who)) return e;
    if (!X || !Y || T <= 0) {
        set_error("%s: null X / Y or T <= 0", who);
        return R97Q_EINVAL;
    }
    if (rank > 0 && (!A || !B || !t_out)) {
        set_error("%s: rank %d needs A, B and t_out", who, (int)rank);
        return R97Q_EINVAL;
    }
    const Shape sh = shape(T, w->rows, w->cols, rank);
    if (int e = check_ws(workspace_bytes, fwd_ws(sh).total, workspace, who)) return e;
    uint8_t* wsb = static_cast<uint8_t*>(workspace);
    const hipStream_t s = (hipStream_t)stream;
    if (int e = fwd_prep(sh, X, A, scale, t_out, wsb, s)) return e;
    return fwd_base(w, sh, B, Y, y_dtype, wsb, s);
}

int r97q_lora_bwd_prep(int64_t T, int64_t N, int64_t K, const uint16_t* dY, const uint16_t* A,
                       const uint16_t* B, const float* t, int32_t rank, float scale, void* workspace,
                       int64_t workspace_bytes, R97IqrStream stream) {
    clear_error();
    const char* who = "r97q_lora_bwd_prep";
    if (int e = shape_ok(T, N, K, who)) return e;
    if (int e = check_rank(rank, who)) return e;
    // t is required with rank > 0: dB's operand is written here, and r97q_lora_bwd_grads cannot
    // tell a workspace without it
    if (!dY || (rank > 0 && (!A || !B || !t))) {
        set_error("%s: null dY, or A, B or t with rank > 0", who);
        return R97Q_EINVAL;
    }
    const Shape sh = shape(T, N, K, rank);
    if (int e = check_ws(workspace_bytes, bwd_ws(sh).total, workspace, who)) return e;
    return bwd_prep(sh, dY, A, B, t, scale, static_cast<uint8_t*>(workspace), (hipStream_t)stream);
}

int r97q_lora_bwd_grads(int64_t T, int64_t N, int64_t K, const uint16_t* X, const uint16_t* dY,
                        int32_t rank, float* dA, float* dB, void* workspace, int64_t workspace_bytes,
                        R97IqrStream stream) {
    clear_error();
    const char* who = "r97q_lora_bwd_grads";
    if (int e = shape_ok(T, N, K, who)) return e;
    if (int e = check_rank(rank, who)) return e;
    if (rank == 0) return R97Q_OK;
    if ((dA && !X) || (dB && !dY)) {
        set_error("%s: dA needs X, dB needs dY", who);
        return R97Q_EINVAL;
    }
    const Shape sh = shape(T, N, K, rank);
    if (int e = check_ws(workspace_bytes, bwd_ws(sh).total, workspace, who)) return e;
    return bwd_grads(sh, X, dY, dA, dB, static_cast<uint8_t*>(workspace), (hipStream_t)stream);
}

int r97q_qlinear_dx_base(const R97qWeight* w, const uint16_t* dY, int64_t T, int32_t rank, void* dX,
                         int32_t dx_dtype, int32_t dx_accumulate, void* workspace,
                         int64_t workspace_bytes, R97IqrStream stream) {
    clear_error();
    const char* who = "r97q_qlinear_dx_base";
    if (int e = check_weight(w)) return e;
    if (int e = check_rank(rank, who)) return e;
    if (!dY || !dX || T <= 0) {
        set_error("%s: null dY / dX or T <= 0", who);
        return R97Q_EINVAL;
    }
    const Shape sh = shape(T, w->rows, w->cols, rank);
    if (int e = check_ws(workspace_bytes, bwd_ws(sh).total, workspace, who)) return e;
    return dx_base(w, sh, dX, dx_dtype, dx_accumulate, static_cast<uint8_t*>(workspace), (hipStream_t)stream);
}

int r97q_qlinear_lora_bwd(const R97qWeight* w, const uint16_t* X, const uint16_t* dY, int64_t T,
                          const uint16_t* A, const uint16_t* B, int32_t rank, float scale,
                          const float* t, void* dX, int32_t dx_dtype, int32_t dx_accumulate,
                          float* dA, float* dB, void* workspace, int64_t workspace_bytes,
                          R97IqrStream stream) {
    clear_error();
    const char* who = "r97q_qlinear_lora_bwd";
    if (int e = check_weight(w)) return e;
    if (int e = check_rank(rank, who)) return e;
    if (!dY || !dX || T <= 0) {
        set_error("%s: null dY / dX or T <= 0", who);
        return R97Q_EINVAL;
    }
    if (rank > 0 && (!A || !B || !t || !X)) {
        set_error("%s: rank %d needs X, A, B and t", who, (int)rank);
        return R97Q_EINVAL;
    }
    const Shape sh = shape(T, w->rows, w->cols, rank);
    if (int e = check_ws(workspace_bytes, bwd_ws(sh).total, workspace, who)) return e;
    uint8_t* wsb = static_cast<uint8_t*>(workspace);
    const hipStream_t s = (hipStream_t)stream;
    if (int e = bwd_prep(sh, dY, A, B, t, scale, wsb, s)) return e;
    // the factor gradients' chunk sums by the gradient launch, added into dA and dB by the dX
    // launch (spread over its workgroups, in chunk order)
    if (rank > 0)
        if (int e = bwd_grads(sh, X, dY, dA, dB, wsb, s, true)) return e;
    return dx_base(w, sh, dX, dx_dtype, dx_accumulate, wsb, s, rank > 0 ? dA : nullptr, rank > 0 ? dB : nullptr);
}

int r97q_gemm_nt_q_dx(const R97qWeight* w, const uint16_t* dY, int64_t T, const float* a_scale, void* dA,
                      int32_t da_dtype, int32_t accumulate, R97IqrStream stream) {
    clear_error();
    const char* who = "r97q_gemm_nt_q_dx";
    if (int e = check_weight(w)) return e;
    if (!dY || !dA || !a_scale || T <= 0) {
        set_error("%s: null dY / dA / a_scale or T <= 0", who);
        return R97Q_EINVAL;
    }
    const Shape sh = shape(T, w->rows, w->cols, 0);
    return dx_scaled(w, sh, dY, dA, da_dtype, accumulate, (hipStream_t)stream, a_scale);
}

int r97q_gemm_nt_q_fwd(const int8_t* codes, const uint16_t* scale, int64_t N, int64_t K, const int8_t* a,
                       const float* a_scale, int64_t T, void* Y, int32_t y_dtype, R97IqrStream stream) {
    clear_error();
    const char* who = "r97q_gemm_nt_q_fwd";
    if (!codes || !scale || !a || !a_scale || !Y) {
        set_error("%s: null codes / scale / a / a_scale / Y", who);
        return R97Q_EINVAL;
    }
    if (T <= 0 || N <= 0 || K <= 0 || N % q::kBN || K % q::kGroup) {
        set_error("%s: T %lld N %lld K %lld (T > 0, N and K multiples of 128)", who, (long long)T, (long long)N,
                  (long long)K);
        return R97Q_EINVAL;
    }
    if (y_dtype != R97Q_F32 && y_dtype != R97Q_BF16) {
        set_error("%s: y_dtype %d (R97Q_F32 or R97Q_BF16)", who, (int)y_dtype);
        return R97Q_EINVAL;
    }
    q::Params p{};
    p.a = a;
    p.a_scale = a_scale;
    p.codes = codes;
    p.scale = scale;
    p.T = T;
    p.N = N;
    p.K = K;
    p.out = Y;
    p.out_f32 = y_dtype == R97Q_F32;
    p.mtiles = (int)((T + q::kBM - 1) / q::kBM);
    p.otiles = (int)(N / q::kBN);
    return q::launch_forward(p, (hipStream_t)stream);
}

int64_t r97q_lora_shrink_q_bwd_workspace_bytes(int64_t T, int64_t K, int32_t rank) {
    return rank_ok(rank) && T > 0 && K > 0 ? shrink_q_ws(T, K, rank).total : -1;
}

int r97q_lora_shrink_q_bwd(int64_t T, int64_t K, const void* a, int32_t a_dtype, const float* a_scale, int64_t groups,
                           int64_t group_width_cols, const uint16_t* A, int32_t rank, const float* t_cot, float* da,
                           float* ds, float* dA, void* workspace, int64_t workspace_bytes, R97IqrStream stream) {
    clear_error();
    const char* who = "r97q_lora_shrink_q_bwd";
    if (T <= 0 || K <= 0 || K % kBN || groups <= 0 || groups > K) {
        set_error("%s: T %lld K %lld groups %lld (T > 0, K a multiple of 128, 0 < groups <= K)", who, (long long)T,
                  (long long)K, (long long)groups);
        return R97Q_EINVAL;
    }
    if (a_dtype != R97Q_I8 && a_dtype != R97Q_F32) {
        set_error("%s: a_dtype %d (R97Q_I8 codes or R97Q_F32 code values)", who, (int)a_dtype);
        return R97Q_EINVAL;
    }
    const int64_t gw = group_width_cols > 0 ? group_width_cols : group_width(K, groups);
    if ((groups - 1) * gw >= K) {
        set_error("%s: %lld groups of %lld columns do not fit K %lld", who, (long long)groups, (long long)gw,
                  (long long)K);
        return R97Q_EINVAL;
    }
    if (int e = check_rank(rank, who)) return e;
    if (rank == 0 || (!da && !ds && !dA)) return R97Q_OK;
    if (!a || !a_scale || !A || !t_cot) {
        set_error("%s: null a, a_scale, A or t_cot", who);
        return R97Q_EINVAL;
    }
    const ShrinkQWs ws = shrink_q_ws(T, K, rank);
    if (int e = check_ws(workspace_bytes, ws.total, workspace, who)) return e;
    uint8_t* wsb = static_cast<uint8_t*>(workspace);
    const hipStream_t s = (hipStream_t)stream;
    const int64_t ldt = grad_ld(T);
    const int code_f32 = a_dtype == R97Q_F32;
    uint16_t* P = reinterpret_cast<uint16_t*>(wsb + ws.P);
    uint16_t* Pt = reinterpret_cast<uint16_t*>(wsb + ws.Pt);
    int* done = reinterpret_cast<int*>(wsb + ws.done);
    if (int e = launch_split(t_cot, T, rank, ldt, 1.0f, P, dA ? Pt : nullptr, done, (int)grad_blocks(K), s)) return e;
    if (da || ds) {
        // g = t_cot . A, then its two code-basis cotangents
        uint16_t* At = reinterpret_cast<uint16_t*>(wsb + ws.At);
        float* g = reinterpret_cast<float*>(wsb + ws.g);
        if (int e = launch_transpose2(nullptr, nullptr, 0, A, At, K, rank, s)) return e;
        if (int e = launch_lora_up(P, At, T, K, rank, g, 0, s)) return e;
        if (int e = launch_coded_cot(g, a, code_f32, a_scale, T, K, groups, gw, da, ds, s)) return e;
    }
    if (dA) {
        // dA += t_cot^T . x with x = [hi | lo](a * a_scale): two gradient passes, one a half
        uint16_t* xhi = reinterpret_cast<uint16_t*>(wsb + ws.xhi);
        uint16_t* xlo = reinterpret_cast<uint16_t*>(wsb + ws.xlo);
        if (int e = launch_coded_x(a, code_f32, a_scale, T, K, groups, gw, xhi, xlo, s)) return e;
        for (const uint16_t* x : {xhi, xlo}) {
            GradArgs g{};
            g.T = T;
            g.ldt = ldt;
            g.chunk = grad_chunk_rows(T, K, 0);
            g.one[0] = GradOne{Pt, x, K, dA, 1.0f, 0, reinterpret_cast<float*>(wsb + ws.part), done};
            if (int e = launch_lora_grads(rank, g, 1, s)) return e;
        }
    }
    return R97Q_OK;
}

int64_t r97q_lora_shrink_bwd_workspace_bytes(int64_t T, int64_t K, int32_t rank) {
    return rank_ok(rank) && T > 0 && K > 0 ? shrink_ws(T, K, rank).total : -1;
}

int r97q_lora_shrink_bwd(int64_t T, int64_t K, const uint16_t* X, const uint16_t* A, int32_t rank,
                         const float* t_cot, float* dX, int32_t dx_accumulate, float* dA, void* workspace,
                         int64_t workspace_bytes, R97IqrStream stream) {
    clear_error();
    const char* who = "r97q_lora_shrink_bwd";
    if (T <= 0 || K <= 0 || K % kBN) {
        set_error("%s: T %lld K %lld (T > 0, K a multiple of 128)", who, (long long)T, (long long)K);
        return R97Q_EINVAL;
    }
    if (int e = check_rank(rank, who)) return e;
    if (rank == 0 || (!dX && !dA)) return R97Q_OK;
    if (!A || !t_cot || (dA && !X)) {
        set_error("%s: null A or t_cot, or dA without X", who);
        return R97Q_EINVAL;
    }
    const ShrinkWs ws = shrink_ws(T, K, rank);
    if (int e = check_ws(workspace_bytes, ws.total, workspace, who)) return e;
    uint8_t* wsb = static_cast<uint8_t*>(workspace);
    const hipStream_t s = (hipStream_t)stream;
    const int64_t ldt = grad_ld(T);
    uint16_t* P = reinterpret_cast<uint16_t*>(wsb + ws.P);
    uint16_t* Pt = reinterpret_cast<uint16_t*>(wsb + ws.Pt);
    uint16_t* At = reinterpret_cast<uint16_t*>(wsb + ws.At);
    int* done = reinterpret_cast<int*>(wsb + ws.done);
    if (int e = launch_split(t_cot, T, rank, ldt, 1.0f, P, dA ? Pt : nullptr, done, (int)grad_blocks(K), s)) return e;
    if (dX) {
        if (int e = launch_transpose2(nullptr, nullptr, 0, A, At, K, rank, s)) return e;
        if (int e = launch_lora_up(P, At, T, K, rank, dX, dx_accumulate, s)) return e;
    }
    if (dA) {
        GradArgs g{};
        g.T = T;
        g.ldt = ldt;
        g.chunk = grad_chunk_rows(T, K, 0);
        g.one[0] = GradOne{Pt, X, K, dA, 1.0f, 0, reinterpret_cast<float*>(wsb + ws.part), done};
        if (int e = launch_lora_grads(rank, g, 1, s)) return e;
    }
    return R97Q_OK;
}

int64_t r97q_lora_expand_bwd_workspace_bytes(int64_t T, int64_t N, int32_t rank) {
    return rank_ok(rank) && T > 0 && N > 0 ? expand_ws(T, N, rank).total : -1;
}

int r97q_lora_expand_bwd(int64_t T, int64_t N, const uint16_t* dY, const uint16_t* B, int32_t rank, float scale,
                         const float* t, float* t_cot, float* dB, void* workspace, int64_t workspace_bytes,
                         R97IqrStream stream) {
    clear_error();
    const char* who = "r97q_lora_expand_bwd";
    if (T <= 0 || N <= 0 || N % kBN) {
        set_error("%s: T %lld N %lld (T > 0, N a multiple of 128)", who, (long long)T, (long long)N);
        return R97Q_EINVAL;
    }
    if (int e = check_rank(rank, who)) return e;
    if (rank == 0 || (!t_cot && !dB)) return R97Q_OK;
    if (!dY || !B || (dB && !t)) {
        set_error("%s: null dY or B, or dB without t", who);
        return R97Q_EINVAL;
    }
    const ExpandWs ws = expand_ws(T, N, rank);
    if (int e = check_ws(workspace_bytes, ws.total, workspace, who)) return e;
    uint8_t* wsb = static_cast<uint8_t*>(workspace);
    const hipStream_t s = (hipStream_t)stream;
    const int64_t ldt = grad_ld(T);
    uint16_t* Bt = reinterpret_cast<uint16_t*>(wsb + ws.Bt);
    uint16_t* Pt2 = reinterpret_cast<uint16_t*>(wsb + ws.Pt2);
    if (int e = launch_transpose2(B, Bt, N, nullptr, nullptr, 0, rank, s)) return e;
    DownArgs a{};
    a.In = dY;
    a.W = Bt;
    a.T = T;
    a.Kin = N;
    a.ldt = dB ? ldt : T;
    a.r = rank;
    a.sa = scale;
    a.sb = scale;
    a.out = t_cot;
    a.out_add = 1;
    a.zero = reinterpret_cast<int*>(wsb + ws.done);
    a.nzero = (int)grad_blocks(N);
    if (dB) {
        a.U2 = t;
        a.s2 = scale;
        a.Pt2 = Pt2;
    }
    if (int e = launch_lora_down(a, s)) return e;
    if (dB) {
        GradArgs g{};
        g.T = T;
        g.ldt = ldt;
        g.chunk = grad_chunk_rows(T, 0, N);
        g.one[0] = GradOne{Pt2, dY, N, dB, 1.0f, 1, reinterpret_cast<float*>(wsb + ws.part),
                           reinterpret_cast<int*>(wsb + ws.done)};
        if (int e = launch_lora_grads(rank, g, 1, s)) return e;
    }
    return R97Q_OK;
}

int64_t r97q_qlinear_lora_fwd_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

int r97q_qlinear_lora_fwd_noalloc(const R97qWeight* w, const uint16_t* X, int64_t T, const uint16_t* A,
                                  const uint16_t* B, int32_t rank, float scale, void* Y, int32_t y_dtype,
                                  float* t_out, R97IqrStream stream) {
    clear_error();
    const char* who = "r97q_qlinear_lora_fwd_noalloc";
    if (int e = check_weight(w)) return e;
    if (int e = check_rank(rank, who)) return e;
    if (!X || !Y || T <= 0) {
        set_error("%s: null X / Y or T <= 0", who);
        return R97Q_EINVAL;
    }
    if (rank > 0 && (!A || !B || !t_out)) {
        set_error("%s: rank %d needs A, B and t_out", who, (int)rank);
        return R97Q_EINVAL;
    }
    const Shape sh = shape(T, w->rows, w->cols, rank);
    const int64_t need = fwd_ws(sh, true).total;
    if (need > kNoAllocScratchBytes) {
        set_error("%s: T %lld x K %lld at rank %d needs %lld workspace bytes, past the %lld this entry holds "
                  "(use r97q_qlinear_lora_fwd with a workspace)",
                  who, (long long)T, (long long)w->cols, (int)rank, (long long)need, (long long)kNoAllocScratchBytes);
        return R97Q_EWORKSPACE;
    }
    uint8_t* wsb = nullptr;
    if (int e = scratch_of_current_device(&wsb, who)) return e;
    const hipStream_t s = (hipStream_t)stream;
    if (int e = fwd_prep(sh, X, A, scale, t_out, wsb, s)) return e;
    return fwd_base(w, sh, B, Y, y_dtype, wsb, s, true);
}

}  // extern "C"

