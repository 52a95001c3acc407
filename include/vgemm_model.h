/*
 * vgemm model files -- the real-weights path of libvgemm.so: the POISDv1 reader and the GEMM weight
 * preparation of the reference's device model, as a C ABI.
 *
 * Replaces, in emanwrxsti/vela:
 *   meow::Poisd (src/poisd.h:10-36, src/poisd.cpp:11-54)   -> vgemm_model_open / _tensor / _name
 *   meow::DevModel::load, ::mergeLins, ::lin, ::norm (src/engine.h:12-13,19-37, src/engine.cu:11-101)
 *                                                          -> vgemm_model_prepare / _upload / _lin / _norm
 *
 * File format (POISDv1, little-endian): "POISDv1\0", u32 tensor count, then per tensor u16 name
 * length, the name bytes, u8 dtype (0 int8, 1 int16, 2 int32, 3 uint8), u8 rank, rank x u32 dims and
 * the row-major data; nothing may follow the last tensor. The file is mapped read-only, not copied.
 *
 * Weight preparation (per int8 rank-2 tensor "<base>.w" that has "<base>.m", except "te.tok.w"):
 * W [N x K] -> [Np x Kp] with Np = N rounded up to 64, Kp = K rounded up to 16, zero padded; 3x3
 * convolutions (base ending ".conv1", ".conv2", "conv_in", "conv_out", "downsamplers.0.conv" or
 * "upsamplers.0.conv") permute K tap-major (column k = c*9 + tap moves to tap*C + c); cst[n] = int4
 * {m, s, b, wsum} with wsum = sum of row n over the real K, pad rows {1, 0, 0, 0}. Merged linears
 * (one GEMM for several projections sharing K): "<blk>.attn1.to_qkv" = [to_q; to_k; to_v],
 * "<blk>.ff.net.0.proj.ag" = [a; g] and "<blk>.ff.net.0.proj.agi" = rows a0, g0, a1, g1, ... (the
 * layout EPI_GEGLU reads) for the UNet's 16 transformer blocks, and "te.layers.<l>.self_attn.qkv"
 * for the text encoder's 23 layers, each built only when all of its parts exist.
 *
 * Host pointers returned by these calls stay valid until vgemm_model_close; device pointers after
 * vgemm_model_upload stay valid until then too (one device allocation holds them all).
 */
#ifndef VGEMM_MODEL_H
#define VGEMM_MODEL_H
#include <stddef.h>
#include <stdint.h>

#include "vgemm.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Model-file errors (cannot open, read error, bad magic, truncated, bad dtype, trailing data,
 * missing tensor): the reference's Poisd::load returns false with these messages. */
enum { VGEMM_ERR_FORMAT = -4 };

/* meow::PoisdTensor dtype codes (src/poisd.h:11) */
enum { VGEMM_DT_I8 = 0, VGEMM_DT_I16 = 1, VGEMM_DT_I32 = 2, VGEMM_DT_U8 = 3 };

typedef struct VgemmModel VgemmModel;

/* meow::PoisdTensor (src/poisd.h:10-16): data points into the mapped file (host memory, possibly
 * unaligned); offset is its byte offset in the file. Ranks above 8 are reported as rank with the
 * first 8 dims. */
typedef struct VgemmTensor {
    int dtype;
    int rank;
    uint32_t dims[8];
    size_t count;
    size_t offset;
    size_t bytes;
    const void* data;
} VgemmTensor;

/* A prepared linear: meow::Lin (src/engine.h:12). w_host / cst_host after vgemm_model_prepare; w /
 * cst (device) after vgemm_model_upload, else NULL. */
typedef struct VgemmLin {
    int N, K, Np, Kp, conv3;
    const int8_t* w_host;     /* [Np x Kp] */
    const int32_t* cst_host;  /* [Np x 4] {m, s, b, wsum} */
    const int8_t* w;
    const int32_t* cst;
} VgemmLin;

/* A normalisation's parameters: meow::Norm (src/engine.h:13): g, beta [C] (Q16 int32) and den (the
 * "<base>.eps" scalar), for every "<base>.g" with "<base>.beta" and "<base>.eps". */
typedef struct VgemmNorm {
    int C;
    int64_t den;
    const int32_t* g_host;
    const int32_t* beta_host;
    const int32_t* g;
    const int32_t* beta;
} VgemmNorm;

/* meow::Poisd::load (src/poisd.cpp:11-54): map and parse `path`, check the structure and the
 * reference's required tensors. On failure *out is NULL and vgemm_last_error() holds the reference's
 * message. (The reference's model hash, a SHA-256, is not computed: that belongs to its consensus
 * layer, outside the GEMM path.) */
int vgemm_model_open(const char* path, VgemmModel** out);
void vgemm_model_close(VgemmModel* model);

/* Poisd::entries() in its order (names sorted bytewise, as std::map): count and i-th name. */
int vgemm_model_count(const VgemmModel* model);
const char* vgemm_model_name(const VgemmModel* model, int i);
/* Poisd::get (src/poisd.cpp:56-58): "missing tensor <name>" if absent. */
int vgemm_model_tensor(const VgemmModel* model, const char* name, VgemmTensor* out);

/* The host half of DevModel::load (src/engine.cu:11-70,87-101): prepare every linear and the merged
 * ones, and gather the normalisations. Host only (no HIP call); idempotent. */
int vgemm_model_prepare(VgemmModel* model);
/* The device half (src/engine.cu:11-70): one hipMalloc on `device` for every prepared W and cst,
 * every norm's g/beta and the int32 tables "lut.phi" and "lut.sigmoid" (256-byte aligned each),
 * filled by synchronous copies. Calls vgemm_model_prepare first if needed. Once per model. */
int vgemm_model_upload(VgemmModel* model, int device);
size_t vgemm_model_device_bytes(const VgemmModel* model);

/* DevModel::lin / ::hasLin / ::norm (src/engine.cu:103-104): "no linear <name>", "no norm <name>". */
int vgemm_model_lin(const VgemmModel* model, const char* name, VgemmLin* out);
int vgemm_model_lin_count(const VgemmModel* model);
const char* vgemm_model_lin_name(const VgemmModel* model, int i);
int vgemm_model_norm(const VgemmModel* model, const char* name, VgemmNorm* out);
/* An int32 table uploaded by vgemm_model_upload ("lut.phi", "lut.sigmoid"): device pointer and
 * element count (DevModel::lutPhi32 / lutSigmoid32, src/engine.h:27). */
int vgemm_model_table(const VgemmModel* model, const char* name, const int32_t** dev, int* count);

#ifdef __cplusplus
}
#endif
#endif
