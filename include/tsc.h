/*
 * tsc.h — C ABI of libtrellis_sparse.so: TRELLIS.2 submanifold sparse conv3d on MI355X (gfx950).
 *
 * Every entry point takes plain pointers and sizes.  Device buffers are raw HIP device addresses
 * (a TS host passes them as u64 / Deno "pointer"; a Python host passes tensor.data_ptr()).
 * Every call returns an int status (TSC_OK == 0); on failure tsc_last_error() holds a message
 * for the calling thread.  All compute calls are enqueue-only on the context's stream and
 * return before the GPU finishes; tsc_sync() waits.
 *
 * Interfaces replaced (reference = johnandersen777/TRELLIS.2-stableprojectorz):
 *   SparseConv3d.forward pass0+pass1 (neighbor map)   src/sparse/ops/conv3d.ts:62-152,
 *        WGSL src/sparse/ops/conv3d_wgsl.ts:44-128;  Python hashmap_fallback (README.md:111)
 *   SparseConv3d.forward pass2 (gather-GEMM-bias)     src/sparse/ops/conv3d.ts:154-221,
 *        WGSL src/sparse/ops/conv3d_wgsl.ts:132-231;  Python conv_none (README.md:109)
 *   layerNorm                                         src/dense/ops/layer_norm.ts:12-125
 *   silu                                              src/dense/ops/silu.ts:11-56
 *   add (residual)                                    src/dense/ops/elementwise.ts:22-65
 *   decoder upsample (1 -> 8 children)                src/models/sparse_unet_vae_decoder.ts:155-175
 *   sparseLinear / ConvNeXt block linears             src/sparse/ops/linear.ts:9-29,
 *                                                     src/models/sparse_unet_vae_decoder.ts:48-78
 *   sparseAttention / scaledDotProductAttention       src/sparse/ops/attention.ts:24-79,
 *                                                     src/dense/ops/attention.ts:36-110
 *   SafetensorsFile + per-tensor upload               src/runtime/weights.ts:58-194,
 *                                                     src/model/loader.ts:134-162
 */
#ifndef TSC_H
#define TSC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TSC_VERSION 5

/* Status codes returned by every entry point. */
enum tsc_status {
  TSC_OK = 0,
  TSC_ERR_INVALID = 1,     /* bad argument: null pointer, bad size, misaligned buffer */
  TSC_ERR_UNSUPPORTED = 2, /* valid request this build does not implement (e.g. kernel 5x5x5) */
  TSC_ERR_HIP = 3,         /* a HIP runtime call failed */
  TSC_ERR_OOM = 4          /* workspace allocation failed */
};

/* Element types of features / weights / outputs.  Accumulation is always fp32. */
enum tsc_dtype { TSC_F32 = 0, TSC_F16 = 1, TSC_BF16 = 2 };

/* Bits the map build ORs into its device status word (0 = map valid). */
#define TSC_MAP_DUPLICATE 1u    /* two rows share one (b,x,y,z) */
#define TSC_MAP_OUT_OF_RANGE 2u /* a coordinate outside [0,B)x[0,X)x[0,Y)x[0,Z) */

/* Neighbor-map construction strategies. */
enum tsc_map_method {
  TSC_MAP_AUTO = 0,   /* occupancy bitmap when the grid is dense enough, else radix sort */
  TSC_MAP_BITMAP = 1, /* occupancy bitmap + popcount rank (a one-pass counting sort) */
  TSC_MAP_RADIX = 2   /* LSD radix sort of packed keys + binary search */
};

/* Epilogues of tsc_conv_fused. */
enum tsc_epilogue {
  TSC_EPI_BIAS = 0,          /* out = conv + bias */
  TSC_EPI_BIAS_RESIDUAL = 1, /* out = conv + bias + residual            (elementwise.ts:22-47) */
  TSC_EPI_BIAS_LN_SILU = 2   /* out = silu(layernorm(conv + bias))      (layer_norm.ts:34-65,
                                                                         silu.ts:25-29) */
};

typedef struct tsc_ctx tsc_ctx;

/* ---- library / context ------------------------------------------------------------------- */
int tsc_version(void);
/* Message of the last failed call on this thread ("" if none).  Valid until the next call. */
const char* tsc_last_error(void);
/* Context bound to one device, enqueueing on `stream` (NULL = the HIP null stream, which is also
 * torch's default stream).  The caller owns the stream.  Not re-entrant: one host thread drives a
 * context at a time. */
int tsc_ctx_create(int device, void* stream, tsc_ctx** out);
int tsc_ctx_destroy(tsc_ctx* ctx);
/* Re-point the context at another stream (e.g. torch.cuda.current_stream()). */
int tsc_ctx_set_stream(tsc_ctx* ctx, void* stream);
void* tsc_ctx_stream(tsc_ctx* ctx);
int tsc_sync(tsc_ctx* ctx);

/* Device memory for hosts without an allocator (the TS host).  Caller frees with tsc_free. */
int tsc_malloc(tsc_ctx* ctx, size_t bytes, void** out);
int tsc_free(tsc_ctx* ctx, void* ptr);
int tsc_memcpy_h2d(tsc_ctx* ctx, void* dst, const void* src, size_t bytes); /* synchronous */
int tsc_memcpy_d2h(tsc_ctx* ctx, void* dst, const void* src, size_t bytes); /* synchronous */
int tsc_memset_zero(tsc_ctx* ctx, void* dst, size_t bytes);               /* stream-ordered */

/* ---- neighbor map ------------------------------------------------------------------------- */
/* Bytes per packed key: 4 if B*X*Y*Z < 2^31, else 8.  Keys are key = ((b*X+x)*Y+y)*Z+z. */
int tsc_map_key_bytes(int32_t B, int32_t X, int32_t Y, int32_t Z);

/* Build the submanifold neighbor map of a coordinate set.
 *   coords      device int32 (N,4) rows [b,x,y,z], 16-byte aligned
 *   kernel      {Kd,Kh,Kw}; only {3,3,3} is supported.  dilation {dD,dH,dW} >= 1.
 *   nbr_out     device int32 (N,27): nbr[n*27+v] = original row of the voxel at
 *               (x+(kd-1)dD, y+(kh-1)dH, z+(kw-1)dW), v = kd*9+kh*3+kw, or -1 when that voxel is
 *               absent or outside [0,X)x[0,Y)x[0,Z).  Row n, tap 13 is n itself.
 *   keys_out    optional device buffer of N keys (tsc_map_key_bytes each): sorted unique keys.
 *   perm_out    optional device int32 (N): perm[i] = original row of the i-th sorted key.
 *   status_dev  device uint32 (1): set to 0, then OR-ed with TSC_MAP_* bits.  Outputs are valid
 *               only when it reads 0.
 * Mirrors conv3d.ts:62-152 (pass0/pass1) and hashmap_fallback (README.md:111) with the batch index
 * in the key (the WGSL grid omits it, conv3d_wgsl.ts:67). */
int tsc_map_build(tsc_ctx* ctx, const int32_t* coords, int64_t N, int32_t B, int32_t X, int32_t Y,
                  int32_t Z, const int32_t kernel[3], const int32_t dilation[3], int32_t method,
                  void* keys_out, int32_t* perm_out, int32_t* nbr_out, uint32_t* status_dev);

/* A measurement call, not part of the conv path: writes the (N,27) int32 table `out` with the
 * radix map build's fill store pattern and nothing else (blocks of 112 consecutive sorted
 * positions, 9 lanes x 12 bytes of each 108-byte row at row rows[i]; rows NULL = i; rows outside
 * [0, N) skipped; the words are (-1, row, -1) per lane).  rows[i] is its only load.  Given the
 * perm_out of tsc_map_build it takes as long as the fill would if finding the neighbors cost
 * nothing: the floor of a neighbor table in the caller's row order.  Stream-ordered.
 * No counterpart in the reference. */
int tsc_map_write_floor(tsc_ctx* ctx, const int32_t* rows, int64_t N, int32_t* out);

/* Row order for tsc_conv / tsc_conv_fused / tsc_resblock: the map's sorted rows (perm, from
 * tsc_map_build; NULL = 0..N-1), sorted inside windows of 262144 consecutive entries by the
 * reflected-binary rank of their 26-bit mask of present neighbors (ties keep the given order),
 * then regrouped inside chunks of 4096 into 256-row tiles of masks contained in a small tap set.
 * The conv kernels skip a tap for a tile of rows only when no row of the tile has that neighbor,
 * so grouped rows skip far more absent (zero) neighbor work than key order does on thin shells.
 * order_out: device int32 (N), a permutation of 0..N-1.  Stream-ordered; uses the context's
 * workspace.
 * No counterpart in the reference: an acceleration structure derived from the neighbor map,
 * meant to be cached beside it (the reference caches the map per tensor, conv3d.ts:144-148). */
int tsc_map_conv_order(tsc_ctx* ctx, const int32_t* nbr, const int32_t* perm, int64_t N,
                       int32_t* order_out);

/* Gather plan for the narrow convs (Ci = 32 in fp16/bf16): rows in 64-row tiles along a Morton
 * (Z-order) curve of the coordinates, each tile's distinct neighbor rows listed once, and a
 * per-(row, tap) slot table into that list.  tsc_conv_planned then gathers each distinct row
 * once per tile instead of once per (row, tap) reference (~1.9 instead of ~9 row reads per
 * output row on a 1-voxel shell).  coords / nbr / B,X,Y,Z as given to tsc_map_build and its
 * output; plan: device buffer of tsc_map_gather_plan_bytes(N) bytes, 256-byte aligned (-1 from
 * tsc_map_gather_plan_bytes means N is out of range).  Stream-ordered; it uses the context's
 * workspace for the curve sort.
 * No counterpart in the reference: an acceleration structure derived from the neighbor map,
 * meant to be cached beside it (the reference caches the map per tensor, conv3d.ts:144-148). */
int64_t tsc_map_gather_plan_bytes(int64_t N);
int tsc_map_gather_plan(tsc_ctx* ctx, const int32_t* coords, const int32_t* nbr, int64_t N,
                        int32_t B, int32_t X, int32_t Y, int32_t Z, void* plan);

/* ---- convolution -------------------------------------------------------------------------- */
/* out[n,co] = bias[co] + sum_{v: nbr[n,v]>=0} sum_ci feats[nbr[n,v],ci] * W[co,v,ci]
 *   feats (N,Ci), weight (Co,3,3,3,Ci), bias (Co) or NULL, out (N,Co): all `dtype`, row-major,
 *   each aligned to its element size; nbr 4-byte aligned.
 *   order: optional device int32 (N) permutation; rows are processed in that order (pass
 *   tsc_map_conv_order's output, or the map's perm_out for spatial locality).  NULL = 0..N-1.
 *   Results do not depend on it.
 *   Wide tiles of 256 rows run in a longest-first order (a schedule computed from nbr and order)
 *   that the context keeps for the next conv with the same nbr, order and N (at most 4
 *   schedules; tsc_map_build, tsc_map_conv_order and tsc_free of either buffer drop them).  A
 *   schedule only decides which block computes which tile, so it never changes a result.
 *   Any Ci >= 1 (Ci * element size <= 65536 bytes) and 1 <= Co <= 65536, as the reference's
 *   bounds-checked shader (conv3d_wgsl.ts:174-196).  The tuned kernels run when Ci * element size
 *   is a multiple of 32 bytes, Co a multiple of 32 and every buffer 16-byte aligned; other
 *   shapes run a generic kernel (zero-padded K tail, masked Co tail), with the same arithmetic.
 * Replaces conv3d.ts:154-221 / conv3d_wgsl.ts:132-231. */
int tsc_conv(tsc_ctx* ctx, int32_t dtype, const void* feats, const void* weight, const void* bias,
             const int32_t* nbr, const int32_t* order, int64_t N, int32_t Ci, int32_t Co, void* out);

/* tsc_conv followed by an epilogue.  residual (N,Co) is read for TSC_EPI_BIAS_RESIDUAL;
 * ln_gamma / ln_beta (Co, dtype, NULL = 1 / 0) and eps for TSC_EPI_BIAS_LN_SILU, which runs
 * inside the conv kernel when one block owns whole rows (fp16/bf16, Ci * 2 > 64 bytes, Co = 64,
 * or Co = 128 / 256 with Ci * 2 a multiple of 64 bytes; 16-byte aligned gamma / beta) and as a
 * LayerNorm row pass after it otherwise; the results are the same bits either way.
 * out may alias residual. */
int tsc_conv_fused(tsc_ctx* ctx, int32_t dtype, const void* feats, const void* weight,
                   const void* bias, const int32_t* nbr, const int32_t* order, int64_t N,
                   int32_t Ci, int32_t Co, int32_t epilogue, const void* residual,
                   const void* ln_gamma, const void* ln_beta, float eps, void* out);

/* tsc_conv_fused that allocates nothing: no hipMalloc / hipFree / allocating library call, for
 * callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid device allocation).  Same arguments, kernels and results (bit for bit) as
 * tsc_conv_fused; the only scratch it needs, the longest-first tile schedule of the 256-row
 * tiles, lives in a static 512 KiB device array per GPU (held until the process ends) instead
 * of the context's growable workspace.  N must not exceed 16777216 rows (65536 tiles of 256;
 * TSC_ERR_INVALID beyond).  Every call on one GPU shares that array: calls that overlap on one
 * device (different streams or contexts) race on it; calls on one stream are ordered.
 * The array's device address is looked up (hipGetSymbolAddress) by the first call on a context.
 * The schedule is built on every call (the cache of tsc_conv_fused would allocate).
 * Per-kernel profiling (tsc_profile_enable) is suspended during the call.
 * No counterpart in the reference. */
int tsc_conv_fused_noalloc(tsc_ctx* ctx, int32_t dtype, const void* feats, const void* weight,
                           const void* bias, const int32_t* nbr, const int32_t* order, int64_t N,
                           int32_t Ci, int32_t Co, int32_t epilogue, const void* residual,
                           const void* ln_gamma, const void* ln_beta, float eps, void* out);

/* tsc_conv_fused with a gather plan (tsc_map_gather_plan of the same coordinate set and map)
 * in place of the row order.  Ci = 32 with Co = 32 or 64 in fp16/bf16 runs the planned
 * kernel; other shapes run the tsc_conv_fused kernels in the plan's row order.  Same results
 * as tsc_conv_fused, bit for bit.  Replaces conv3d.ts:154-221 for the decoder's narrow convs. */
int tsc_conv_planned(tsc_ctx* ctx, int32_t dtype, const void* feats, const void* weight,
                     const void* bias, const int32_t* nbr, const void* plan, int64_t N,
                     int32_t Ci, int32_t Co, int32_t epilogue, const void* residual,
                     const void* ln_gamma, const void* ln_beta, float eps, void* out);

/* ---- row ops (the ResBlock's epilogue semantics) ------------------------------------------ */
/* y = (x-mean)/sqrt(var+eps)*gamma+beta per row of C, fp32 math; optional SiLU after it.
 * gamma/beta NULL = 1/0.  y may alias x (in place, as layer_norm.ts:12-125). */
int tsc_layernorm(tsc_ctx* ctx, int32_t dtype, const void* x, int64_t N, int32_t C,
                  const void* gamma, const void* beta, float eps, int32_t apply_silu, void* y);
/* y = x * sigmoid(x) elementwise, fp32 math (silu.ts:25-29).  y may alias x. */
int tsc_silu(tsc_ctx* ctx, int32_t dtype, const void* x, int64_t numel, void* y);
/* y = a + b elementwise, fp32 math (elementwise.ts:33-40).  y may alias a. */
int tsc_add(tsc_ctx* ctx, int32_t dtype, const void* a, const void* b, int64_t numel, void* y);

/* Sparse ResBlock: out = x + conv2(silu(LN(conv1(x)+b1))) + b2, with C=Ci=Co.
 * LN uses eps and gamma/beta (NULL = 1/0).  out must not overlap x (TSC_ERR_INVALID if any
 * byte of the two (N,C) ranges is shared).  The intermediate (N,C)
 * activation lives in the context's workspace. */
int tsc_resblock(tsc_ctx* ctx, int32_t dtype, const void* x, const int32_t* nbr,
                 const int32_t* order, int64_t N, int32_t C, const void* w1, const void* b1,
                 const void* ln_gamma, const void* ln_beta, float eps, const void* w2,
                 const void* b2, void* out);

/* ---- per-voxel linear layer ---------------------------------------------------------------- */
/* out (N,Cout) = x (N,Cin) * weight^T + bias (+ residual); weight (Cout,Cin) as nn.Linear, bias
 * (Cout) or NULL, residual (N,Cout) or NULL (it may be out itself; any other overlap of out with
 * residual or with x is TSC_ERR_INVALID).  All `dtype`, fp32
 * accumulation, one hipBLASLt GEMM (bias epilogue, residual as its C operand).  The first call
 * of a shape on a context times the library's candidate algorithms (into scratch rows, so an
 * in-place residual is not applied twice) and synchronizes the stream once; later calls only
 * enqueue.
 * Replaces sparseLinear (src/sparse/ops/linear.ts:9-29) and the matmul + add pairs of the sparse
 * ConvNeXt block (src/models/sparse_unet_vae_decoder.ts:48-78). */
int tsc_linear(tsc_ctx* ctx, int32_t dtype, const void* x, int64_t N, int32_t Cin,
               const void* weight, const void* bias, const void* residual, int32_t Cout, void* out);

/* ---- subdivision (the decoder's upsample step) --------------------------------------------- */
/* Children of every voxel at twice the resolution: parent row n = [b,x,y,z] gives the rows
 * [b, 2x+dx, 2y+dy, 2z+dz], c = dx*4 + dy*2 + dz, each with a copy of the parent's feature row.
 * Rows are parent-major, children in increasing c.  With keep (device uint8 (N); bit c of keep[n]
 * = keep child c of parent n) only the kept children are written, in the same order.
 *   coords      device int32 (N,4), 16-byte aligned, x,y,z < 2^30
 *   feats       device (N,C) `dtype` rows, or NULL for coordinates only
 *   coords_out  device int32 (M,4), feats_out (M,C): M = 8N without keep, else the number of set
 *               bits of keep (tsc_subdivide_count; it synchronizes the stream to return it).
 *               Non-null whenever N > 0 (a host with M == 0 has nothing to call for).
 * Replaces the upsample step of the sparse decoder (src/models/sparse_unet_vae_decoder.ts:155-175,
 * where the TS port only doubles the spatial shape); the spatial shape and the scale of the
 * result are twice the input's. */
int tsc_subdivide_count(tsc_ctx* ctx, const uint8_t* keep, int64_t N, int64_t* count);
int tsc_subdivide(tsc_ctx* ctx, const int32_t* coords, int64_t N, int32_t dtype, const void* feats,
                  int32_t C, const uint8_t* keep, int32_t* coords_out, void* feats_out);

/* ---- varlen attention ---------------------------------------------------------------------- */
/* Scaled-dot-product attention over packed variable-length sequences:
 *   out[n,h,:] = softmax_m(q[n,h,:] . k[m,h,:] * scale) v[m,h,:]
 * for n in [cu_seqlens_q[b], cu_seqlens_q[b+1]) and m in [cu_seqlens_kv[b], cu_seqlens_kv[b+1]),
 * b < B.  A sequence with no keys gives zeros; rows of out outside [cu_seqlens_q[0],
 * cu_seqlens_q[B]) are not written (the Python host zero-fills them, as the reference's zero-
 * initialised output does, attention.ts:49).
 *   q, out (total_q, num_heads, head_dim), k, v (total_kv, num_heads, head_dim): `dtype`,
 *     row-major, 16-byte aligned; out must not alias an input.  head_dim 64 or 128.
 *   cu_seqlens_q / cu_seqlens_kv  device int32 (B+1), non-decreasing, within [0, total]
 *     (values outside are clamped, so a malformed array cannot read out of bounds).
 *   scale  <= 0 means 1/sqrt(head_dim) (attention.ts:64).  max_seqlen_q sizes the grid (longer
 *     sequences are still covered, at a lower parallelism).
 * bf16/f16 on v_mfma 32x32x16 with fp32 softmax and accumulation (P rounded to the input type
 * for the second product); f32 on v_mfma 32x32x2f32.
 * Replaces sparseAttention (src/sparse/ops/attention.ts:24-79: B > 1 as a per-sample CPU round
 * trip) and, with B = 1, scaledDotProductAttention (src/dense/ops/attention.ts:36-110). */
int tsc_attention(tsc_ctx* ctx, int32_t dtype, const void* q, const void* k, const void* v,
                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_kv, int32_t B,
                  int64_t total_q, int64_t total_kv, int32_t num_heads, int32_t head_dim,
                  float scale, int32_t max_seqlen_q, void* out);

/* ---- safetensors weight files -------------------------------------------------------------- */
/* Element types of a safetensors header ("dtype" strings).  F32/F16/BF16 equal TSC_F32/F16/BF16. */
enum tsc_st_dtype {
  TSC_ST_F32 = 0, TSC_ST_F16 = 1, TSC_ST_BF16 = 2, TSC_ST_F64 = 3, TSC_ST_I64 = 4, TSC_ST_I32 = 5,
  TSC_ST_I16 = 6, TSC_ST_I8 = 7, TSC_ST_U8 = 8, TSC_ST_BOOL = 9, TSC_ST_U16 = 10, TSC_ST_U32 = 11,
  TSC_ST_U64 = 12, TSC_ST_F8_E4M3 = 13, TSC_ST_F8_E5M2 = 14
};
/* out_dtype of tsc_st_load that copies the stored bytes unchanged. */
#define TSC_ST_RAW (-1)

typedef struct tsc_st tsc_st;
/* Opens a .safetensors file and parses its header only (8-byte little-endian length + JSON);
 * tensor data stays on disk until loaded.  Rejects malformed headers, unknown dtypes, duplicate
 * names and data offsets that disagree with shape x dtype or lie outside the file.
 * Replaces SafetensorsFile.open (src/runtime/weights.ts:67-99). */
int tsc_st_open(const char* path, tsc_st** out);
int tsc_st_close(tsc_st* f);                                       /* weights.ts:188-192 */
/* Number of tensors and of __metadata__ entries, and the file offset of the data block
 * (SafetensorsHeader.tensors.size / metadata / dataByteOffset, weights.ts:18-22, 106-108). */
int tsc_st_counts(tsc_st* f, int64_t* tensors, int64_t* metadata, int64_t* data_offset);
/* Name of tensor `index` in header order, NUL-terminated into name[name_len]
 * (listTensors, weights.ts:111-113). */
int tsc_st_name(tsc_st* f, int64_t index, char* name, int32_t name_len);
/* Metadata entry `index` (header order) as NUL-terminated key and value (weights.ts:94). */
int tsc_st_metadata(tsc_st* f, int64_t index, char* key, int32_t key_len, char* value,
                    int32_t value_len);
/* dtype (tsc_st_dtype), rank, shape (up to max_dims entries) and data_offsets [begin, end)
 * relative to the data block of a tensor; any output may be NULL (getTensorInfo,
 * weights.ts:120-123).  Unknown names are TSC_ERR_INVALID. */
int tsc_st_info(tsc_st* f, const char* name, int32_t* dtype, int32_t* ndim, int64_t* shape,
                int32_t max_dims, int64_t* offsets);
/* Streams one tensor from the file into device memory dst on the context's stream.
 *   out_dtype TSC_ST_RAW (or the stored float type): the stored bytes unchanged (readTensorRaw,
 *             weights.ts:125-142); dst holds end - begin bytes.
 *   out_dtype TSC_F32 / TSC_F16 / TSC_BF16 from a stored F32, F16 or BF16 tensor: converted on the
 *             GPU, numel elements of out_dtype.  To F32 this is readTensorF32 bit for bit
 *             (weights.ts:150-177: BF16 bits << 16; F16 IEEE widening, NaN -> sign|0x7fc00000);
 *             to F16/BF16 round to nearest even, NaN -> sign | canonical quiet NaN.
 *             Other stored types must be loaded raw (TSC_ERR_UNSUPPORTED).
 * Returns once the last chunk is queued: work later on the same stream sees the tensor; the host
 * waits with tsc_sync.  Replaces the per-tensor upload of loadModelWeights
 * (src/model/loader.ts:134-162, getTensor). */
int tsc_st_load(tsc_ctx* ctx, tsc_st* f, const char* name, int32_t out_dtype, void* dst);

/* ---- per-kernel timing -------------------------------------------------------------------- */
/* While enabled, every kernel the context launches is bracketed by hipEvents on its stream.
 * tsc_profile_collect syncs the stream and folds the pending launches into per-kernel totals
 * (count of distinct kernel names in *count); tsc_profile_entry reads one total. */
int tsc_profile_enable(tsc_ctx* ctx, int on);
int tsc_profile_collect(tsc_ctx* ctx, int* count);
int tsc_profile_entry(tsc_ctx* ctx, int index, char* name, int name_len, double* total_ms,
                      int64_t* launches);
int tsc_profile_reset(tsc_ctx* ctx);

#ifdef __cplusplus
}
#endif

#endif /* TSC_H */
