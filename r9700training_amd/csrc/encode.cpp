// encode.cpp -- an IQR trellis quantizer for the trunk form (trellis.mad, per-row f32 scale plus a
// per-128-column scale.col factor), host C++, threaded.
//
// The reference's quantizer is radiance's libquant grid_tcq (absent from the reference tree), so
// this is this repo's own: its output is a valid stored weight that the reference's decode reads
// (src/iqr_decode.h), which is what every parity check pins; its quantization error is reported,
// not matched.
//
// Scales: scale.col[kb] = rms of the block's 128 columns over rms of the whole weight; the row
// scale = rms of the row divided by the codebook's rms (so the codes' targets have the codebook's
// spread); the effective scale of (row, block) is bf16(row * factor), the decode's fold
// (src/iqr_form.h:203-216). Codes: for each column and each tail-biting run, a greedy walk down
// the rows picks, at each row, the code whose state value is nearest the row's target given the
// codes above it. The run's seam (the first rows read the last rows' codes) is settled by walking
// twice more with the previous walk's last codes as the seam and keeping the walk with the
// smallest error as the decode will actually see it (the wrapped states recomputed exactly).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/r97q.h"

namespace {

uint16_t to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

float from_bf16(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

int32_t mad_value(uint32_t st, uint32_t a, uint32_t b) {
    const uint32_t h = ((st & 0xFFFFFFu) * (a & 0xFFFFFFu) + b) & 0x3F3F3F3Fu;
    return (int32_t)((h & 0xFFu) + ((h >> 8) & 0xFFu) + ((h >> 16) & 0xFFu) + (h >> 24)) - 126;
}

struct Job {
    const float* Wt;  // [K, N]: the weight transposed, so a column walk is sequential
    int64_t N, K;
    int bits, L, run;
    const int8_t* lut;
    const float* eff;  // [N, K/128] effective scale
    uint32_t* codes;   // [K, N] unpacked
};

// Walk rows [r0, r1) of column k with `seam` as the codes above r0 (oldest first, c-1 of them);
// returns the squared error of the walk as the decode would read it with that seam.
double walk(const Job& j, int64_t k, int64_t r0, int64_t r1, const uint32_t* seam, uint32_t* out) {
    const int c = (j.L + j.bits - 1) / j.bits;
    const uint32_t mask = (1u << j.L) - 1u;
    uint32_t st = 0;
    for (int q = 0; q < c - 1; ++q) st = ((st << j.bits) | seam[q]) & mask;
    const int nc = 1 << j.bits;
    double err = 0.0;
    for (int64_t r = r0; r < r1; ++r) {
        const float s = j.eff[r * (j.K / 128) + k / 128];
        const float u = s > 0.0f ? j.Wt[k * j.N + r] / s : 0.0f;
        const uint32_t base = (st << j.bits) & mask;
        int best = 0;
        float be = 3.4e38f;
        for (int cc = 0; cc < nc; ++cc) {
            const float d = (float)j.lut[base | (uint32_t)cc] - u;
            const float e = d * d;
            if (e < be) {
                be = e;
                best = cc;
            }
        }
        out[r - r0] = (uint32_t)best;
        st = base | (uint32_t)best;
        err += (double)be * s * s;
    }
    return err;
}

// The error of codes[r0, r1) of column k as the decode reads them (seam = the run's own tail).
double decode_error(const Job& j, int64_t k, int64_t r0, int64_t r1, const uint32_t* codes) {
    const int c = (j.L + j.bits - 1) / j.bits;
    const uint32_t mask = (1u << j.L) - 1u;
    const int64_t len = r1 - r0;
    double err = 0.0;
    for (int64_t r = r0; r < r1; ++r) {
        uint32_t st = 0;
        for (int q = c - 1; q >= 0; --q) {
            int64_t t = r - q;
            if (t < r0) t += len;
            st = ((st << j.bits) | codes[t - r0]) & mask;
        }
        const float s = j.eff[r * (j.K / 128) + k / 128];
        const float d = (float)j.lut[st] * s - j.Wt[k * j.N + r];
        err += (double)d * d;
    }
    return err;
}

void encode_column(const Job& j, int64_t k) {
    const int c = (j.L + j.bits - 1) / j.bits;
    std::vector<uint32_t> a(j.run), best(j.run);
    std::vector<uint32_t> seam(c > 1 ? c - 1 : 1, 0);
    for (int64_t r0 = 0; r0 < j.N; r0 += j.run) {
        const int64_t r1 = std::min(r0 + (int64_t)j.run, j.N);
        const int64_t len = r1 - r0;
        std::fill(seam.begin(), seam.end(), 0u);
        double best_err = -1.0;
        for (int pass = 0; pass < 3; ++pass) {
            walk(j, k, r0, r1, seam.data(), a.data());
            const double e = decode_error(j, k, r0, r1, a.data());
            if (best_err < 0.0 || e < best_err) {
                best_err = e;
                std::copy(a.begin(), a.begin() + len, best.begin());
            }
            for (int q = 0; q < c - 1; ++q) seam[q] = a[len - (c - 1) + q];
        }
        for (int64_t r = r0; r < r1; ++r) j.codes[k * j.N + r] = best[r - r0];
    }
}

}  // namespace

extern "C" {

// Quantize W [N, K] (host f32, row-major) to the trunk IQR form. Outputs (host):
//   codes     [N, ceil(K*bits/8)] bytes, codes packed LSB first along each row
//   row_scale [N] f32 (the `scale` plane, one a row)
//   col_factor[K/128] f32 (the `scale.col` plane)
// mad_a / mad_b: the trellis.mad codebook. threads <= 0: hardware concurrency.
// Returns 0, or R97Q_EINVAL for a shape or form outside bits 1..8, L 1..24, K % 128, run >= c.
int r97q_iqr_encode_trellis(const float* W, int64_t N, int64_t K, int32_t bits, int32_t state_bits,
                            int32_t run_rows, uint32_t mad_a, uint32_t mad_b, uint8_t* codes,
                            float* row_scale, float* col_factor, int32_t threads, double* rel_err) {
    if (!W || !codes || !row_scale || !col_factor || N <= 0 || K <= 0 || K % 128) return R97Q_EINVAL;
    if (bits < 1 || bits > 8 || state_bits < 1 || state_bits > 24 || run_rows < 1) return R97Q_EINVAL;
    const int c = (state_bits + bits - 1) / bits;
    if (run_rows < c || (N % run_rows != 0 && N % run_rows < c)) return R97Q_EINVAL;
    const int64_t nkb = K / 128;
    // the codebook and its spread
    std::vector<int8_t> lut((size_t)1 << state_bits);
    double vv = 0.0;
    for (size_t st = 0; st < lut.size(); ++st) {
        lut[st] = (int8_t)mad_value((uint32_t)st, mad_a, mad_b);
        vv += (double)lut[st] * lut[st];
    }
    const double code_rms = std::sqrt(vv / (double)lut.size());
    // scales
    double tot = 0.0;
    std::vector<double> blk(nkb, 0.0);
    for (int64_t n = 0; n < N; ++n) {
        double rs = 0.0;
        for (int64_t k = 0; k < K; ++k) {
            const double w = W[n * K + k];
            rs += w * w;
            blk[k / 128] += w * w;
        }
        tot += rs;
        row_scale[n] = (float)(std::sqrt(rs / (double)K) / code_rms);
    }
    const double all_rms = std::sqrt(tot / (double)(N * K));
    for (int64_t kb = 0; kb < nkb; ++kb)
        col_factor[kb] = all_rms > 0 ? (float)(std::sqrt(blk[kb] / (double)(N * 128)) / all_rms) : 1.0f;
    std::vector<float> eff((size_t)(N * nkb));
    for (int64_t n = 0; n < N; ++n)
        for (int64_t kb = 0; kb < nkb; ++kb)
            eff[(size_t)(n * nkb + kb)] = from_bf16(to_bf16(row_scale[n] * col_factor[kb]));
    // codes, column by column
    std::vector<uint32_t> raw((size_t)(N * K));
    std::vector<float> Wt((size_t)(N * K));
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) Wt[(size_t)(k * N + n)] = W[n * K + k];
    Job j{Wt.data(), N, K, bits, state_bits, run_rows, lut.data(), eff.data(), raw.data()};
    int T = threads > 0 ? threads : (int)std::max(1u, std::thread::hardware_concurrency());
    std::vector<std::thread> pool;
    for (int t = 0; t < T; ++t)
        pool.emplace_back([&, t]() {
            for (int64_t k = t; k < K; k += T) encode_column(j, k);
        });
    for (auto& th : pool) th.join();
    // pack
    const int64_t rb = (K * bits + 7) / 8;
    std::memset(codes, 0, (size_t)(N * rb));
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
            const uint64_t o = (uint64_t)k * bits;
            const uint32_t v = raw[(size_t)(k * N + n)];
            for (int b = 0; b < bits; ++b)
                if (v >> b & 1u) codes[n * rb + (int64_t)((o + b) >> 3)] |= (uint8_t)(1u << ((o + b) & 7));
        }
    if (rel_err) {
        // relative RMS error of the decoded weight (the decode's own seam)
        double num = 0.0;
        for (int64_t k = 0; k < K; ++k)
            for (int64_t r0 = 0; r0 < N; r0 += run_rows) {
                const int64_t r1 = std::min(r0 + (int64_t)run_rows, N);
                num += decode_error(j, k, r0, r1, raw.data() + k * N + r0);
            }
        *rel_err = tot > 0 ? std::sqrt(num / tot) : 0.0;
    }
    return R97Q_OK;
}

}  // extern "C"
