// det_gguf.h -- the GGUF container det's weights live in, and `det convert` (host code in libdet_hip.so).
//
// Replaces crates/det/src/gguf.rs (reader over a memory map, header writer) and crates/det/src/convert.rs +
// config.rs (`det convert --no-calibrate`: a float qwen35 GGUF -> a det GGUF) for callers of this library.
// Tensor types: F32 (0), F16 (1), BF16 (30) and det's quantized linears DET_W4/6/8 (0xDE04/0xDE06/0xDE08), whose
// data are det rows [codes][c f32][m u16 x K/128] (gguf.rs:79-138).  Errors do not abort: NULL or -1 is returned
// and det_gguf_last_error() says why (the reference returns io::Error, gguf.rs:208-300).
#pragma once
#include <stdint.h>
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif

typedef struct det_gguf det_gguf;

// GGUF metadata value types (gguf.rs:60-75)
enum { DET_GGUF_U8 = 0, DET_GGUF_I8, DET_GGUF_U16, DET_GGUF_I16, DET_GGUF_U32, DET_GGUF_I32, DET_GGUF_F32,
       DET_GGUF_BOOL, DET_GGUF_STR, DET_GGUF_ARRAY, DET_GGUF_U64, DET_GGUF_I64, DET_GGUF_F64 };

const char* det_gguf_last_error(void);           // message of the last failed call on this thread

// Gguf::open (gguf.rs:208-300): magic "GGUF", version 2 or 3, metadata, tensor table; data start aligned to
// general.alignment (default 32); every tensor must be of a known type, at most 2-D, and fit the file.
det_gguf* det_gguf_open(const char* path);
void      det_gguf_close(det_gguf* g);
uint64_t  det_gguf_data_start(const det_gguf* g);
uint64_t  det_gguf_alignment(const det_gguf* g);

// metadata, in file order
uint64_t    det_gguf_n_kv(const det_gguf* g);
const char* det_gguf_kv_key(const det_gguf* g, uint64_t i);
uint32_t    det_gguf_kv_type(const det_gguf* g, uint64_t i);
int64_t     det_gguf_find_kv(const det_gguf* g, const char* key);                // index or -1
// Value::as_u64 / as_f32 / as_str (gguf.rs:27-55): 1 and *out set when the key exists and converts, else 0
int         det_gguf_get_u64(const det_gguf* g, const char* key, uint64_t* out);
int         det_gguf_get_f32(const det_gguf* g, const char* key, float* out);
const char* det_gguf_get_str(const det_gguf* g, const char* key);                // NULL if absent or not a string
// arrays: element type and length; element j as u64 / f64 / string where it converts (1), else 0 / NULL
int         det_gguf_get_array(const det_gguf* g, const char* key, uint32_t* elem_type, uint64_t* len);
int         det_gguf_array_u64(const det_gguf* g, const char* key, uint64_t j, uint64_t* out);
int         det_gguf_array_f64(const det_gguf* g, const char* key, uint64_t j, double* out);
const char* det_gguf_array_str(const det_gguf* g, const char* key, uint64_t j);

// tensors, in file order (TensorInfo, gguf.rs:160-190): dims in ggml order (dims[0] fastest, the row length)
uint64_t    det_gguf_n_tensors(const det_gguf* g);
int64_t     det_gguf_find_tensor(const det_gguf* g, const char* name);           // index or -1
const char* det_gguf_tensor_name(const det_gguf* g, uint64_t i);
uint32_t    det_gguf_tensor_type(const det_gguf* g, uint64_t i);
int         det_gguf_tensor_dims(const det_gguf* g, uint64_t i, uint64_t dims[4]);  // returns the rank
uint64_t    det_gguf_tensor_offset(const det_gguf* g, uint64_t i);                 // from the data start
uint64_t    det_gguf_tensor_bytes(const det_gguf* g, uint64_t i);
const void* det_gguf_tensor_data(const det_gguf* g, uint64_t i);                   // inside the mapping

// `det convert <src> --out <dst> [--bits spec] [--rope-positions n] --no-calibrate` (convert.rs:170-402,
// main.rs:517-524): src may be the first of a split set (-00001-of-000NN).  bits = NULL takes
// "6,output=8,ssm_alpha=8,ssm_beta=8"; rope_positions <= 0 takes <arch>.context_length (default 32768).
// Linears are quantized on the GPU (det_quantize_rows), bit-identical to quantize.rs.  0 on success, -1 on error.
int det_convert(const char* src, const char* dst, const char* bits, int64_t rope_positions);

#ifdef __cplusplus
}
#endif
