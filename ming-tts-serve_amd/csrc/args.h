// Plain argument blocks shared by the host glue and the kernels (no device
// code, so host-only translation units can include it).
#pragma once

#include <stdint.h>

namespace ming {

// Weights of one linear as the kernels see them.
struct LinearDev {
    int32_t kind;  // 0 bf16, 1 affine 4-bit / group 64
    int32_t N, K;
    float gscale;
    const uint32_t* w;   // affine: u32 [N, K/8]; bf16: bf16 [N, K] viewed as u32 pairs
    const uint16_t* s;   // bf16 [N, K/64]
    const uint16_t* b;   // bf16 [N, K/64]
};

// fused.LmLayer (src/ming_fused.zig:576-589) as the kernels see it.
struct LayerDev {
    const uint16_t *ln1, *ln2;
    LinearDev q, k, v, o, g, u, d;
    const uint16_t *bq, *bk, *bv;
};

// Everything one decode step touches.  Activations of every layer are kept
// (x[l] is layer l's input, x[n_layers] the stack output), which also lets
// tests read any intermediate.
struct StepArgs {
    const LayerDev* layers;   // device array [n_layers] (persistent schedule)
    int n_layers, H, heads, kvh, hd, I;
    float eps, log2_theta;
    const uint16_t* final_norm;
    LinearDev head;           // tied LM head [V, H]
    LinearDev embed;          // embedding table [V, H]
    uint16_t* kc;             // [n_layers][kvh][cap][hd]
    uint16_t* vc;
    int cap;
    int pos;                  // position of this token (= cached length before the step)
    const int32_t* token_in;  // device id, or null: x[0] already holds the input row
    int32_t* argmax_out;      // device i32, or null
    // Activations of layer l: input x + l*sx, output xo + l*sx, x1 + l*sx,
    // att + l*sx, qkv + l*sq, hh + l*sh.  The stack uses one buffer per layer
    // (xo = x + H, so x[l + 1] is layer l's output); a single-layer call
    // passes caller buffers with zero strides.
    uint16_t* x;
    uint16_t* xo;
    uint16_t* x1;
    uint16_t* att;
    uint16_t* qkv;
    uint16_t* hh;
    int64_t sx, sq, sh;
    float* part;              // attention partials [kvh][nsplit][grp][hd + 2]
    int split_len;            // positions per attention split (multiple of 64)
    uint16_t* hidden;         // [H] final-normed hidden (bf16)
    float* logits;            // [V] f32, or null
    float* amax_v;            // [kMaxParts] argmax partials
    int32_t* amax_i;
    int32_t* flags;           // [0] error flag, [1] grid barrier counter
    // Tagged hand-off buffers of the persistent schedule: u64 words holding a
    // pair of bf16 values (low half) and the step's epoch (high half).
    uint64_t* tx;             // [n_layers + 1][H/2]   layer inputs / stack output
    uint64_t* tq;             // [n_layers][(H + 2*kvh*hd)/2]
    uint64_t* ta;             // [n_layers][H/2]       merged attention
    uint64_t* tx1;            // [n_layers][H/2]
    uint64_t* th;             // [n_layers][I/2]
    int32_t* counters;        // [n_layers * kvh] attention arrivals, [1] head arrivals, [n_layers * kvh] attention
                              // arrivals of XCD-local splits (L2 atomics)
    uint32_t epoch;
    uint64_t* tstamp;         // optional [n_stamps][grid] wall-clock stamps per stage boundary
    // Hubs of the persistent schedule (one workgroup per XCD): each publishes
    // the staged GEMV input of every stage into memory that the other
    // workgroups of its XCD read through their shared L2.
    int nhubs;                // 0: every workgroup stages its own inputs
    int hub_stages;           // stages whose inputs come from the hubs (HUB_* bits); the others stage their own
    uint32_t* img;            // [kMaxHubs][kImgSlots][img_stride] stage images
    int img_stride;           // u32 words per image slot
    uint32_t* hflag;          // [kMaxHubs][nflag] epoch of each published image
    int nflag;                // flag words per hub (>= 4 * n_layers + 1)
    uint64_t* hubtab;         // [kMaxHubs] tagged XCC id of each hub, then [kAttXlSlots] of attention workers
    // Attention splits grouped by XCD (1): worker W-1-(8 sp + g) runs split sp of kv
    // head g, so a kv head's splits share an XCD when workgroup b runs on XCD b % 8
    // (checked per launch); they then meet through that XCD's L2.  0: splits in
    // unit order across the grid, meeting device-coherently.
    int att_xl;
    // XCD-local schedule: o_proj partials of each kv head and down partials of
    // each XCD slot, f32 whose lowest mantissa bit carries the epoch's parity
    // (the reader clears it); xslots = slots that hold SwiGLU groups (and so
    // down partials).  Every word is written at every step of this schedule,
    // and consecutive steps of it use epochs of opposite parity.
    uint32_t* tpo;            // [n_layers][kvh][H]
    uint32_t* tpd;            // [n_layers][8][H]
    int xslots;
    uint64_t* tpa;            // [n_layers][kvh][xnsm][grp][hd + 2] attention split partials, tagged words
    int xnsm;                 // split slots per (layer, kv head) in tpa
    int xloc;                 // 1: hand-offs inside an XCD slot use plain stores where the slot is on one XCD
};

constexpr int kAttXlBase = 32;    // hubtab index of the attention workers' XCC ids
constexpr int kAttXlSlots = 256;
constexpr int kXcdBase = kAttXlBase + kAttXlSlots;  // hubtab index of every workgroup's XCC id (XCD-local schedule)
constexpr int kXcdSlots = 1024;

// Stages of the persistent schedule, as bits of StepArgs::hub_stages.
enum : int { HUB_QKV = 1, HUB_O = 2, HUB_UP = 4, HUB_DOWN = 8, HUB_HEAD = 16 };

// One DiT block (fused.Block, src/ming_fused.zig:482-500): bf16 [out, in]
// linears with biases, two RMSNorm weights; D = hidden, F = feed-forward.
struct DitBlockDev {
    int D, F, heads, hd;
    float eps;
    const uint16_t *norm1, *norm2;
    const uint16_t *wq, *wk, *wv, *wo, *w1, *w2;
    const uint16_t *bq, *bk, *bv, *bo, *b1, *b2;
};

constexpr int kMaxHubs = 8;
constexpr int kImgSlots = 5;  // q/k/v, o_proj, gate/up, down, LM head

constexpr int kMaxParts = 4096;

// ---- VAE decoder GEMM (vae.hip) ----------------------------------------------
// Weight formats and epilogues of the f32 GEMM.
enum VWf : int { VW_BF16 = 0, VW_Q4 = 1, VW_F32 = 2 };
enum VEpi : int {
    VE_PLAIN = 0,   // y = acc (+ bias)
    VE_QKV = 1,     // y = acc + bias, rope on columns < rope_cols (heads of 64, position = row)
    VE_RES = 2,     // y = res + acc
    VE_SWIGLU = 3,  // y = (g * sigmoid(g)) * u, g from w0, u from w1
    VE_WIN = 4,     // y = acc * win[col]
};

// One weight of the f32 GEMM: bf16 [n][K], MLX affine 4-bit (u32 [n][K/8] +
// bf16 scales/biases [n][K/64]) or f32 [n][K].
struct VSeg {
    const void* w;
    const uint16_t *s, *b;
    float gs;               // affine global scale
    const uint16_t* bias;   // bf16 [n] or null (VE_PLAIN, VE_QKV)
    int n;                  // output columns (a multiple of 64 except in the last segment)
    int rope;               // VE_QKV: 1 = rotary on these columns (heads of 64, position = row)
};

// C [M][N] = A [M][K] (f32) x W^T; the output columns are the segments'
// columns one after another (N = sum of seg[i].n).  ks > 1 splits K into ks
// slices whose partials [ks][M][N] (f32, in part) a reduce kernel sums in
// slice order before the epilogue.
struct VGemm {
    const float* a;
    int lda, M, K;
    VSeg seg[3];
    int nseg;
    VSeg up;                // VE_SWIGLU: the up weight over seg[0]'s columns
    const float* res;       // VE_RES: f32 [M][ldres]
    int ldres;
    const float* win;       // VE_WIN: f32 [N]
    float* y;
    int ldy;
    float log2_theta;
    int ks;
    float* part;
};

}  // namespace ming
