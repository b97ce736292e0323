/* mgr.h — C entry points of the MI355X MaskGIT transformer runtime (lib/libmg_hip.so).
 *
 * A model handle owns a GGUF file (mg::Model::load), a HipRuntime and the graph context; a
 * forward builds the reference's transformer graph (mg::build_transformer,
 * src/mg-transformer.cpp:32-111) for the given tokens and runs it on the GPU — the path of
 * the reference's TransformerFwd hook (include/mg-generate.hpp:15, tools/main.cpp:122-130).
 * Status codes: 0 = OK, negative = error with mgr_last_error() set (per thread).
 */
#ifndef MGR_H
#define MGR_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mgr_model mgr_model;

/* algo: 0 = default (2), 1 = int8-dot FC, 2 = dequantized weights x fp16 activations (the
 * reference's choice on a device without cl_arm_integer_dot_product, mg-opencl.cpp:1237-1238) */
int mgr_load(const char* gguf_path, int device, int algo, mgr_model** out);
void mgr_free(mgr_model* m);
const char* mgr_last_error(void);
/* n_layer, n_head, n_embd, head_dim, vocab_size, n_positions, mask_token_id */
int mgr_hparams(const mgr_model* m, int32_t out[7]);
const char* mgr_device_name(const mgr_model* m);
/* decoding parameters: image positions, VQGAN codebook size, default choice temperature
 * (maskgit.n_tokens, maskgit.vqgan.codebook_size, maskgit.sampling.choice_temperature) */
int mgr_decode_params(const mgr_model* m, int32_t* n_tokens, int32_t* codebook, float* choice_temperature);

/* tokens [B][S] (I32) -> logits [B][S][vocab_size] (fp32, host). logits may be NULL: the
 * forward then runs without the final readback. */
int mgr_forward(mgr_model* m, const int32_t* tokens, int S, int B, float* logits);

/* A named node of the last mgr_forward or mgr_decode_images graph (embd_post_norm, blk.<l>.attn_post,
 * blk.<l>.ffn_post, output_norm, output_logits: src/mg-transformer.cpp:47, 91, 98, 106, 109),
 * as the reference's verification tools read them: its values are current only if that
 * forward ran with MG_DUMP_NAMED set in the environment, which makes the runtime read every
 * named node back (mg-opencl.cpp:1627-1641). Copies up to `capacity` floats into out (NULL:
 * size query); returns the element count, or < 0. */
int mgr_named(const mgr_model* m, const char* name, float* out, int64_t capacity);

/* Iterative decoding of B images on the device: the reference's generate() loop
 * (src/mg-generate.cpp:39-121) without the VQGAN decode. Image b starts from class token
 * class_ids[b] + codebook and all n_tokens positions masked, draws from
 * std::mt19937_64(seeds[b]) in the reference's order and runs `steps` transformer forwards,
 * each followed by the on-device sampling / confidence / re-mask step (mgh_decode_step); the
 * logits never leave HBM. temperature < 0 selects the model's choice temperature.
 * out_tokens [B][n_tokens] receives the final grid (the reference's result without the
 * class token, the input of its VQGAN decode). */
int mgr_generate(mgr_model* m, const int32_t* class_ids, const uint64_t* seeds, int B, int steps,
                 float temperature, int32_t* out_tokens);

/* The VQGAN decode of B token grids: grids [B][n_tokens] (I32 codebook ids, row-major h*L + w
 * of the L x L latent grid) -> images [B][3][side][side] (fp32, channel planes, w innermost: the
 * reference's image layout ne = {W, H, 3, 1} per image). The graph is the reference's decoder
 * (mg::build_vqgan_decoder, src/mg-vqgan.cpp:62-110), the computation of its VqganFwd hook
 * (include/mg-generate.hpp:17, tools/main.cpp:137-152), here for B images in one graph.
 * images may be NULL: the decode then runs without the readback. The images are decoded in
 * groups of 8 (an image's result does not depend on its group). Each GroupNorm, conv (+ bias)
 * and res-block output is named after its weights' prefix (res blocks: "<prefix>.out"; the
 * inputs of conv_in and of each up-sampling conv: "<prefix>.in") for mgr_named, whose values
 * are those of the last group. */
int mgr_decode_images(mgr_model* m, const int32_t* grids, int B, float* images);
/* side of the decoded images: sqrt(n_tokens) * 2^(levels - 1); 0 if the model has no VQGAN */
int mgr_image_side(const mgr_model* m);

/* The reference's whole generate() (src/mg-generate.cpp:39-123) for B images: mgr_generate's
 * device-resident decoding, then the VQGAN decode of the final grids (mgr_decode_images, in
 * groups of 8 images). images [B][3][side][side] as mgr_decode_images; out_tokens
 * [B][n_tokens] receives the grids (may be NULL). */
int mgr_generate_images(mgr_model* m, const int32_t* class_ids, const uint64_t* seeds, int B, int steps,
                        float temperature, int32_t* out_tokens, float* images);

/* per-op device-time profile of the following forwards (each node timed on its own) */
int mgr_profile_enable(mgr_model* m, int on);
/* writes up to cap rows "name count ms\n" into buf (NUL-terminated) */
int mgr_profile_report(const mgr_model* m, char* buf, size_t cap);

/* ---- host-only inspection (no device needed) ---- */
/* parse a GGUF file: hparams as in mgr_hparams, and the tensor count */
int mgr_gguf_info(const char* gguf_path, int32_t hparams_out[7], int64_t* n_tensors);
/* build the forward graph for S x B tokens and count its nodes per op code
 * (counts[op] for op in 0..31, mg::Op values); returns the node count or < 0 */
int mgr_graph_stats(const char* gguf_path, int S, int B, int32_t counts[32]);

#ifdef __cplusplus
}
#endif
#endif /* MGR_H */
