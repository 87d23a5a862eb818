// Argument block and buffer geometry of the persistent flow head (one launch
// per cfmSample, cfm_persistent.hip), shared by the host glue and the kernel.
#pragma once

#include <stdint.h>

namespace ming {

// The shape the persistent flow head is built for: the reference's DiT
// (hidden 1024, 16 heads of 64, ff 4096), 2 CFG halves x 3 positions, a
// latent of 64 (src/ming_model.zig:37-41, :1161-1203).
constexpr int kPD = 1024, kPF = 4096, kPR = 6, kPL = 3, kPHeads = 16, kPHd = 64, kPLat = 64;
constexpr int kPMaxBlocks = 16;
constexpr int kPSteps = 10;        // Euler steps (flowSchedule)
constexpr int kPXcds = 8;          // one head workgroup per XCD
constexpr int kPMinWorkers = 220;  // 7 compute waves each: the 1536 q/k/v row pairs in one round

// u32 words of one XCD's stage images: A (the rms1 rows, raw), A's half-row
// sums of squares, B (attention rows), C (the rms2 rows, raw), C's half-row
// sums, D (ff1 rows)
constexpr int kPImgA = 0;
constexpr int kPImgAp = kPImgA + kPR * kPD / 2;
constexpr int kPImgB = kPImgAp + 16;
constexpr int kPImgC = kPImgB + kPR * kPD / 2;
constexpr int kPImgCp = kPImgC + kPR * kPD / 2;
constexpr int kPImgD = kPImgCp + 16;
constexpr int kPImgWords = kPImgD + kPR * kPF / 2;
constexpr int kPFlagLine = 32;     // slice flags of one image (u32 each)

// tagged words {bf16 pair, epoch} per (Euler step, block)
constexpr int kPTq = 3 * kPR * kPD / 2;  // q | k | v rows
constexpr int kPTx = kPR * kPD / 2;      // x1 rows; block output rows
constexpr int kPTh = kPR * kPF / 2;      // ff1 rows

struct CfmPBlock {
    const uint16_t *norm1, *norm2;
    const uint16_t *wq, *wk, *wv, *wo, *w1, *w2;
    const uint16_t *bq, *bk, *bv, *bo, *b1, *b2;
};

struct CfmPArgs {
    const CfmPBlock* blocks;  // device [nblk]
    int nblk, steps, nflag;   // nflag = steps * nblk * 4 (image flags per hub)
    float eps;
    const float *cos_t, *sin_t;       // rotary [L][hd / 2]
    const uint16_t* te;               // t_emb [steps][2][D]
    const uint16_t* ce;               // c_emb(z) rows [2][D]
    const uint16_t* xh;               // x_emb(history) [D]
    const uint16_t *wx, *bx;          // x_embedder [D][latent], [D]
    const uint16_t *fnorm, *wf, *bf;  // final layer: norm [D], linear [latent][D], bias [latent]
    const uint16_t *noise, *sde, *dt, *sq;  // y_0 [latent]; sde [steps][latent]; dt, sqrt|dt| [steps]
    float cfg, shift;
    uint16_t* y_out;                  // [latent]
    uint16_t* y_steps;                // optional [steps][latent]
    uint64_t *tq, *tx1, *th, *txo;    // tagged outputs, [steps * nblk][kPTq | kPTx | kPTh | kPTx]; tq and th
                                      // unit-major: [q | k | v][kPD / 2] and [kPF / 2] column pairs, then kPR rows
    uint32_t* img;                    // [kPXcds][kPImgWords] stage images, one set per XCD
    uint32_t* flg;                    // [kPXcds][4][kPFlagLine] slice flags
    uint64_t* xcctab;                 // [kPXcds]: {XCC id of head x, epoch}
    uint64_t* tstamp;                 // optional [6][nflag] wall-clock stamps
    // tags of this launch: epoch for the stage outputs and the XCC table,
    // epoch + f for the slice flags of image f (f < nflag); every tag exceeds
    // every earlier launch's
    uint32_t epoch;
    int32_t* flags;                   // [0] a bounded wait expired
};

}  // namespace ming
