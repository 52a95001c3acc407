/*
 * vgemm engine blocks -- the reference engine's resnet and transformer blocks on the kernels of
 * libvgemm.so, as a C ABI: the composition of the GEMMs with the integer GroupNorm / LayerNorm, the
 * exact attention and the elementwise kernels that one UNet block runs, bit-exact.
 *
 * Replaces, in emanwrxsti/vela:
 *   meow::Engine (src/engine.h:58-116), its arena (src/engine.h:38-44) and configuration
 *   (src/engine.h:56, EngineConfig: fusedAttention, fusedLoader and customGemmMaxK at their defaults,
 *   gnFuse selectable)                                       -> vgemm_engine_create / _destroy
 *   Engine::resnet (src/engine.cu:389-405)                   -> vgemm_engine_resnet
 *   Engine::transformer (src/engine.cu:406-454)              -> vgemm_engine_transformer
 *   the cross-attention K/V of Engine::setPrompt (src/engine.cu:540-560), one block at a time, from a
 *   context of B samples                                     -> vgemm_engine_set_context
 *
 * Activations are NHWC int32 rows [B * T x C] (meow::Tensor, src/engine.h:36) in caller-owned device
 * memory; the blocks' intermediates come from the engine's arena, one device allocation made by
 * vgemm_engine_create, released at the end of each block (as the reference's arena marks do). Every
 * block call is asynchronous on `stream`, allocates nothing and may be captured into a graph
 * (vgemm_graph_begin / _end); calls on one engine must not overlap.
 */
#ifndef VGEMM_ENGINE_H
#define VGEMM_ENGINE_H
#include <stddef.h>
#include <stdint.h>

#include "vgemm.h"
#include "vgemm_model.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct VgemmEngine VgemmEngine;

/* meow::Tensor (src/engine.h:36): d [B * T x C] int32; rowmax (optional, [B * T]): the per-row max |x|
 * its producer wrote; gnst (optional, VgemmGnStat [B * 32]): the GroupNorm sum/min/max its producer
 * accumulated. */
typedef struct VgemmActivation {
    int32_t* d;
    int B, T, C;
    uint32_t* rowmax;
    void* gnst;
} VgemmActivation;

/* Engine::Engine for an uploaded model (vgemm_model_upload): arena_bytes of device memory on the
 * current device (hipMalloc, once) for the blocks' intermediates; gn_fuse = EngineConfig::gnFuse
 * (GroupNorm statistics gathered by the producing GEMM's epilogue where the reference would). */
int vgemm_engine_create(const VgemmModel* model, size_t arena_bytes, int gn_fuse, VgemmEngine** out);
void vgemm_engine_destroy(VgemmEngine* engine);
/* the arena's high-water mark so far (Engine::arenaPeak, src/engine.h:69) */
size_t vgemm_engine_arena_peak(const VgemmEngine* engine);

/* Engine::resnet (src/engine.cu:389-405) of the block "<prefix>" (linears <prefix>.conv1, .conv2 and
 * optionally .conv_shortcut, norms <prefix>.norm1, .norm2) on x [B, H * W, C]: out->d [B * H * W x N]
 * (caller-allocated, N = conv2's outputs). out->gnst, when not NULL (VgemmGnStat [B * 32], caller
 * memory), receives the GroupNorm records of the output where the reference gathers them (gn_fuse and
 * a fusable shape: the engine initialises and fills them), else is set to NULL. x->gnst, when not
 * NULL, holds the records of x its producer gathered (they replace k_gn_stats1 for norm1). */
int vgemm_engine_resnet(VgemmEngine* engine, void* stream, const VgemmActivation* x, int H, int W, const char* prefix,
                        VgemmActivation* out);

/* The cross-attention K/V of transformer block "<block>" (= "<prefix>.transformer_blocks.0") from a
 * context ctx [B, Tc, Cc] (one row block per sample; the reference replicates one prompt's): the
 * linears <block>.attn2.to_k / .to_v, k_quant_heads and k_quant_v. Kept (in memory the engine owns)
 * until the next call for the same block or vgemm_engine_destroy. Not capturable (allocates on first
 * use of a block). */
int vgemm_engine_set_context(VgemmEngine* engine, void* stream, const VgemmActivation* ctx, const char* block, int heads);

/* Engine::transformer (src/engine.cu:406-454) of "<prefix>" with `heads` heads of 64 on x [B, T, C]:
 * out->d [B * T x C] (caller-allocated); out->gnst and x->gnst as for vgemm_engine_resnet. Needs
 * vgemm_engine_set_context for its block first, with the same B. */
int vgemm_engine_transformer(VgemmEngine* engine, void* stream, const VgemmActivation* x, const char* prefix, int heads,
                             VgemmActivation* out);

#ifdef __cplusplus
}
#endif
#endif
