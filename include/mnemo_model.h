/*
 * mnemo_model.h -- the split model directory the reference engine loads, read on the host
 * and placed in device memory for the kernels of this library.
 *
 * Files (MnemoCUDA docs/model-format.md:1-128; loader src/engine.c:376-460, 524-736, 860-890):
 *   config.json             GGUF metadata, architecture prefix auto-detected
 *   resident_manifest.json  {"tensors": [{"name", "offset", "size", "type_id", "dims"}, ...]}
 *   resident_weights.bin    the non-expert tensors at those offsets
 *   expert_manifest.json    optional: per layer {"expert_size", "gate_size", "up_size",
 *                           "down_size"} under the layer number as a string key
 *   experts/layer_XX.bin    n_experts records [gate][up][down] of expert_size bytes
 *
 * On one MI355X everything is resident: mnemo_model_upload copies the resident tensors into
 * one device buffer (each tensor 256-byte aligned, as src/engine.c:872-875) and every
 * expert layer into its own device array, the layout mnemo_moe_decode / mnemo_moe_prefill
 * take (experts + e * expert_size + {0, gate_size, gate_size + up_size}).  Files are read
 * in bounded chunks through a pinned staging buffer.  The reference's NVMe expert cache,
 * heat map and tokenizer are the caller's business and are not read here.
 *
 * All functions return 0 or an MNEMO_ERR_* code and record a message for
 * mnemo_last_error_string().  Parsing and validation do not touch the GPU.
 */
#ifndef MNEMO_MODEL_H
#define MNEMO_MODEL_H

#include <stddef.h>

#include "mnemo_kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    char prefix[32];  /* qwen3moe, qwen35moe, glm4moe, qwen3next, llama or qwen2 */
    int hidden_size, n_layers, n_heads, n_kv_heads, head_dim;
    int eff;          /* expert_feed_forward_length */
    int n_experts, experts_per_tok, context_length, full_attention_interval, vocab_size;
    float rope_theta, rms_eps;
} mnemo_model_config;

typedef struct {
    char name[128];
    size_t offset, size;   /* in resident_weights.bin */
    int type_id;
    int n_dims;
    long long dims[4];
} mnemo_tensor_info;

typedef struct {
    size_t expert_size, gate_size, up_size, down_size;
    int down_type_id;      /* mnemo_down_type_id(down_size, hidden, eff) */
    int n_experts;
} mnemo_expert_layer_info;

/* config.json text -> cfg.  Required: {prefix}.embedding_length, .block_count,
 * .attention.head_count, .attention.head_count_kv; the rest default as in
 * src/engine.c:411-444 (vocab from tokenizer.ggml.tokens_count or vocab_size, else 151936). */
int mnemo_parse_config(const char *json_text, mnemo_model_config *cfg);
/* resident_manifest.json text -> up to max entries; *n receives the number of tensors. */
int mnemo_parse_resident_manifest(const char *json_text, mnemo_tensor_info *out, int max, int *n);
/* expert_manifest.json text: the sizes of layer `layer` (0 where absent). */
int mnemo_parse_expert_manifest(const char *json_text, int layer, mnemo_expert_layer_info *info);
/* Q4_K / Q6_K / F32 bytes of one row of n values (0 for other types). */
size_t mnemo_row_bytes(int type_id, int n);

typedef struct mnemo_model mnemo_model;

/* Reads and validates the directory: every tensor inside resident_weights.bin, every
 * experts/layer_XX.bin of size n_experts * expert_size, gate + up + down <= expert_size. */
int mnemo_model_open(const char *dir, mnemo_model **out);
const mnemo_model_config *mnemo_model_config_of(const mnemo_model *m);
int mnemo_model_n_tensors(const mnemo_model *m);
int mnemo_model_tensor_at(const mnemo_model *m, int i, mnemo_tensor_info *info);
/* Layers with an expert file; info of layer `layer` (MNEMO_ERR_BAD_ARG if it has none). */
int mnemo_model_expert_layer(const mnemo_model *m, int layer, mnemo_expert_layer_info *info);
/* Device copies on the current device (experts too when with_experts != 0). */
int mnemo_model_upload(mnemo_model *m, int with_experts);
/* Device pointer of a tensor by name (after upload); NULL-safe outputs. */
int mnemo_model_tensor(const mnemo_model *m, const char *name, mnemo_tensor_info *info, void **dev_ptr);
/* Device array of a layer's experts (after upload with experts). */
int mnemo_model_experts(const mnemo_model *m, int layer, void **dev_ptr);
/* Frees the device copies and the host state. */
void mnemo_model_close(mnemo_model *m);

#ifdef __cplusplus
}
#endif
#endif /* MNEMO_MODEL_H */
