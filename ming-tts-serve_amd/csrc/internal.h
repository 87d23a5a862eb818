// Host-side internals shared by the C-ABI glue and the kernel launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "../../include/ming_hip.h"
#include "args.h"
#include "batch.h"

namespace ming {
// Device memory owned by a context or model; grows on demand.
struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
    hipError_t ensure(size_t n) {
        if (n <= bytes) return hipSuccess;
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
        hipError_t e = hipMalloc(&p, n);
        if (e == hipSuccess) bytes = n;
        return e;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
};
}  // namespace ming

struct ming_ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;     // own_stream or a borrowed one
    std::string err;
    int32_t* dev_flags = nullptr;     // [0] device-side error flag (spin timeout)
    int num_cus = 0;
    size_t max_lds = 0;
    bool alive = false;
    ming::DevBuf part;                // attention partials of ming_lm_layer
    ming::DevBuf qstage;              // staged activations of ming_qgemm
    bool timeout_seen = false;        // ming_sync saw the device error flag
    bool exclusive = false;           // caller keeps the device to this context's work
    void* scratch = nullptr;          // this device's fixed scratch array (scratch.hip), or null
};

namespace ming {

int set_err(ming_ctx* ctx, int status, const std::string& msg);

// ---- fixed device scratch (scratch.hip) ----
// Bytes of the per-device array; scratch_init resolves the current device's
// copy once (at context creation), scratch_ptr returns it (null before).
size_t scratch_bytes();
hipError_t scratch_init(int device);

// gelu's tanh table (tanh_tab.h) into the DiT kernels' device arrays of
// `device` (current), once per device.
hipError_t tanh_tables_init(int device);
void* scratch_ptr(int device);
int hip_check(ming_ctx* ctx, hipError_t e, const char* what);

// ---- launchers (return hipError_t of the launch) ----
hipError_t launch_qgemv(hipStream_t st, int M, const uint16_t* x, const uint32_t* w, const uint16_t* s,
                        const uint16_t* b, int N, int K, float gscale, uint16_t* y_bf16, float* y_f32);
// Gathered 4-bit product (qgemv.hip): y[p] = g * x[lhs[p]] W[rhs[p]]^T for
// P pairs; x bf16 [Bx][M][K], W [E] MLX-affine matrices [N][K]; an index out
// of range raises flags[2].  gather_vectors(K): activation vectors one
// workgroup stages at once (M must not exceed it).
int gather_vectors(int K);
hipError_t launch_gather_qmm(hipStream_t st, const uint16_t* x, const uint32_t* w, const uint16_t* s,
                             const uint16_t* b, const int32_t* lhs, const int32_t* rhs, int P, int Bx, int E, int M,
                             int N, int K, float gscale, bool sorted, int32_t* flags, uint16_t* y_bf16, float* y_f32);
hipError_t launch_dequantize(hipStream_t st, const uint32_t* w, const uint16_t* s, const uint16_t* b, int64_t N,
                             int64_t K, float gscale, uint16_t* out);
hipError_t launch_quantize(hipStream_t st, const uint16_t* w, int64_t N, int64_t K, float gscale, uint32_t* wq,
                           uint16_t* s, uint16_t* b);
// ---- batched decode (qgemm.hip, batch.hip) ----
// Batched 4-bit GEMM on MFMA over activations staged by launch_stage; a.blocks
// is filled by the launcher.  epi is a QEpi.
hipError_t launch_qgemm_epi(hipStream_t st, QgemmArgs a, int epi);
// Per-row argmax of n rows from the wide GEMM's partials [n][nblk]
// (nblk = qgemm_argmax_blocks: the column blocks of the launch for that shape,
// at most ceil(N / 32)).
int qgemm_argmax_blocks(int M, int K, int N);
hipError_t launch_argmax_partials(hipStream_t st, const float* pmax, const int32_t* pidx, int nblk, int n,
                                  int32_t* out);
// Rows [0, Mp) of x [M][ldx] (Mp = M rounded up to 16; rows >= M zero) staged
// group-major as uint4 xs [K/64][Mp][8] + f32 xsum [K/64][Mp]; norm_w
// non-null: rms first.
hipError_t launch_stage(hipStream_t st, const uint16_t* x, int ldx, int M, int K, const uint16_t* norm_w, float eps,
                        void* xs, float* xsum, uint16_t* hout, int32_t* pos_inc);
hipError_t launch_embed_rows(hipStream_t st, const LinearDev& E, const int32_t* tokens, int n, uint16_t* x);
hipError_t launch_rope_table(hipStream_t st, float* cs, int max_ctx, int half, float log2_theta);
hipError_t launch_paged_attn(hipStream_t st, const PagedAttnArgs& a, int n_seq);
hipError_t launch_merge_stage(hipStream_t st, const MergeArgs& a);
// rows [n][pps] = n copies of table [pps]; pos [n] = p0, p0 + 1, ...
// Positions [p0, p0 + n) of the pages 0, 1, 2, ... (head_dim 64) into a
// contiguous [n_layers][kvh][cap][64] cache.
hipError_t launch_pages_to_rows(hipStream_t st, const uint16_t* kp, const uint16_t* vp, int n_layers, int kvh,
                                int n_pages, int p0, int n, uint16_t* kc, uint16_t* vc, int cap);
hipError_t launch_prefill_rows(hipStream_t st, const int32_t* table, int pps, int n, int p0, int32_t* rows,
                               int32_t* pos);

// ---- flow head over many sequences (dit.hip, dit_batch.hip) ----
int stop_prob_impl(ming_ctx* ctx, const ming_linear* head, const void* bias, const void* z, float* p_dev,
                   bool with_flags);
uint16_t* lm_input_row(ming_lm_model* m);
int cfm_sample_impl(ming_ctx* ctx, ming_cfm_model* m, const void* z, const void* hist, const void* noise,
                    const void* sde, float cfg, float sigma, float temperature, void* latent_out, void* y_steps,
                    bool pre_done);
int cfm_pre(ming_ctx* ctx, ming_cfm_model* m, const void* z, const void* hist, const ming_linear* stop_head,
            const void* stop_bias, float* p_out);
hipError_t launch_dit_attn(hipStream_t st, const uint16_t* qkv, int B, int L, int D, int heads, int hd, uint16_t* att);
hipError_t launch_dit_block_gemm(hipStream_t st, const DitBlockDev& w, const uint16_t* x, int R, int L,
                                 const float* cos_t, const float* sin_t, uint16_t* hn, uint16_t* qkv, uint16_t* att,
                                 uint16_t* x1, uint16_t* hh, uint16_t* out, float* part, bool hn_ready = false,
                                 const DitBlockDev* next = nullptr);
hipError_t launch_dit_linear_gemm(hipStream_t st, const uint16_t* x, int R, const uint16_t* w, int N, int K,
                                  const uint16_t* b, uint16_t* out);
hipError_t launch_cfm_rows_batch(hipStream_t st, const uint16_t* te, const uint16_t* ce, const uint16_t* bc,
                                 const uint16_t* xh, const uint16_t* xe, int n, int D, uint16_t* rows);
hipError_t launch_cfm_final_batch(hipStream_t st, const uint16_t* h, int n, int L, int D, const uint16_t* norm,
                                  float eps, const uint16_t* wf, const uint16_t* bf, int latent, const uint16_t* y,
                                  const uint16_t* dt, const uint16_t* sq, const uint16_t* sde, int step, int steps,
                                  float cfg, float shift, uint16_t* hn, uint16_t* y_out, uint16_t* y_steps);

// Read-only view of a prepared decode stack (for the batched step).
struct LmView {
    ming_lm_cfg cfg;
    const LayerDev* layers;   // host array [n_layers]
    LinearDev head, embed;
    const uint16_t* final_norm;
};
bool lm_model_view(const ming_lm_model* m, LmView& v);

// ---- VAE decoder (vae.hip) ----
hipError_t launch_vgemm(hipStream_t st, const VGemm& g, int wf, int epi);
hipError_t launch_vrms(hipStream_t st, const float* x, int M, int K, const uint16_t* w, float eps, float* out);
hipError_t launch_vattn(hipStream_t st, const float* qkv, int M, int ldq, int H, int heads, int kvh, int window,
                        float scale, float* att);
hipError_t launch_vup(hipStream_t st, const float* y, const uint16_t* bias, int q4, int T, int C, int scale,
                      float* x);
hipError_t launch_vspec(hipStream_t st, const float* p, int F, int nfft, int ld, float* spec);
hipError_t launch_vola(hipStream_t st, const float* fr, int F, int nfft, int hop, const float* win, float* wave);
hipError_t launch_vwiden(hipStream_t st, const uint16_t* x, int64_t n, float* y);
// Weight views and checks shared with the LM glue (api.cpp).
LinearDev linear_dev(const ming_linear& l);
int check_linear_w(ming_ctx* ctx, const ming_linear& l, int N, int K, const char* name);

}  // namespace ming
