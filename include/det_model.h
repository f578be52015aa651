// det_model.h -- a det GGUF model on the GPU (host code in libdet_hip.so): the reference's Model (crates/det/src/
// model.rs:164-548) and qwen35::forward (qwen35.rs:8-172) over the kernels of det_hip.h.
//
// Load reads the file through the GGUF reader (det_gguf.h), checks every float is finite (model.rs:13-44), uploads
// the norms, rope tables and per-layer vectors, fuses each projection's consecutive same-type same-K tensors into
// one linear (model.rs:180-197) repacked by det_linear_repack, and allocates the KV caches (int8 keys, int16 values)
// and Gated DeltaNet states.  The embedding rows are dequantized on the host from the mapped file, as the
// reference does (model.rs:390-414).  All work runs on det_hip_stream().  Errors do not abort: NULL or -1 is
// returned and det_model_last_error() says why.
#pragma once
#include <stdint.h>
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif

typedef struct det_model det_model;

const char* det_model_last_error(void);

// Model::load (model.rs:164-368): max_ctx positions, batches of at most max_batch tokens
det_model* det_model_load(const char* path, int max_ctx, int max_batch);
void       det_model_free(det_model* m);
int        det_model_vocab(const det_model* m);
int        det_model_pos(const det_model* m);      // positions consumed so far
// Model::reset (model.rs:378-388): position 0, zero GDN states (the KV rows are overwritten as positions refill)
void       det_model_reset(det_model* m);
// Model::forward (model.rs:442-466): ids (1 .. max_batch of them) at the current position; afterwards the logits
// of the last one are the model's logits.  0, or -1 (state untouched) on an empty or oversized batch, a position
// past the context or an id outside the embedding table.
int        det_model_forward(det_model* m, const int* ids, int n);
// Model::prefill (model.rs:499-509): ids in batches of max_batch
int        det_model_prefill(det_model* m, const int* ids, int n);
// the last forward's logits ([vocab] fp32) to host memory; 0 or -1
int        det_model_logits(det_model* m, float* out);
// Model::pick with greedy sampling (model.rs:474-497, Backend::argmax): the lowest index of the largest logit
int        det_model_argmax(det_model* m);
// Model::generate with greedy sampling (model.rs:511-548): prefill prompt, then up to n_new tokens into out,
// stopping after the first id in stop[0 .. n_stop).  Returns the number of tokens written, or -1.
int        det_model_generate(det_model* m, const int* prompt, int n_prompt, int n_new, const int* stop, int n_stop,
                              int* out);

#ifdef __cplusplus
}
#endif
