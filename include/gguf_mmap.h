// gguf_mmap.h -- read-only GGUF v3 file mapping: the subset of CowboyTim/rocm-hip's src/gguf_mmap.h that the MoE
// expert loader (moe_gguf.h) and its callers use, with the same names, argument meaning and error values.
//
// A file is mapped read-only and parsed once: its key/value metadata and tensor table are kept, tensor data stays
// in the mapping. A model split as <prefix>-00001-of-0000N.gguf (llama.cpp's naming) is opened by its first file
// and reads as one tensor table. Every header read is bounds-checked against the file size: a truncated or
// corrupted file fails to open (NULL) instead of being read past its end, and a tensor whose data would lie past
// the end of its file has no data pointer (gguf_get_tensor_ptr returns NULL).

#ifndef GGUF_MMAP_H
#define GGUF_MMAP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gguf_model gguf_model_t;

// Replace src/gguf_mmap.h:15-17. open: NULL when the file is missing, is not GGUF version 3, is corrupted, or is
// one part of a split model other than the first (the reason: gguf_last_error). get_tensor: the tensor's bytes
// in the mapping and their count, NULL for an unknown name or a NULL out_bytes.
gguf_model_t* gguf_mmap_open(const char* path);
void gguf_mmap_close(gguf_model_t* model);
const void* gguf_mmap_get_tensor(const gguf_model_t* model, const char* name, size_t* out_bytes);

// Replace src/gguf_mmap.h:20-30. ne: the tensor's 4 dimensions (ne[d >= n_dims] == 1). Sizes are (size_t)-1 for a
// type whose block layout is not known; the offset is relative to the tensor's file's data section.
int64_t gguf_n_tensors(const gguf_model_t* model);
const char* gguf_tensor_name(const gguf_model_t* model, int64_t idx);
int gguf_tensor_type(const gguf_model_t* model, int64_t idx);
int64_t* gguf_tensor_ne(const gguf_model_t* model, int64_t idx);
uint8_t gguf_tensor_dims(const gguf_model_t* model, int64_t idx);
size_t gguf_tensor_block_size(const gguf_model_t* model, int64_t idx);
size_t gguf_tensor_type_size(const gguf_model_t* model, int64_t idx);
uint64_t gguf_tensor_offset(const gguf_model_t* model, int64_t idx);
size_t gguf_tensor_nbytes(const gguf_model_t* model, int64_t idx);

// Replace src/gguf_mmap.h:33-47: key/value metadata by index; the getters return 0, or -1 on a type mismatch.
int64_t gguf_n_kv(const gguf_model_t* model);
const char* gguf_kv_key(const gguf_model_t* model, int64_t idx);
int gguf_kv_type(const gguf_model_t* model, int64_t idx);
int32_t gguf_kv_get_u8(const gguf_model_t* model, int64_t idx, uint8_t* out);
int32_t gguf_kv_get_i8(const gguf_model_t* model, int64_t idx, int8_t* out);
int32_t gguf_kv_get_u16(const gguf_model_t* model, int64_t idx, uint16_t* out);
int32_t gguf_kv_get_i16(const gguf_model_t* model, int64_t idx, int16_t* out);
int32_t gguf_kv_get_u32(const gguf_model_t* model, int64_t idx, uint32_t* out);
int32_t gguf_kv_get_i32(const gguf_model_t* model, int64_t idx, int32_t* out);
int32_t gguf_kv_get_f32(const gguf_model_t* model, int64_t idx, float* out);
int32_t gguf_kv_get_u64(const gguf_model_t* model, int64_t idx, uint64_t* out);
int32_t gguf_kv_get_i64(const gguf_model_t* model, int64_t idx, int64_t* out);
int32_t gguf_kv_get_f64(const gguf_model_t* model, int64_t idx, double* out);

// Replace src/gguf_mmap.h:50-52: general.alignment (32 when absent), the first file's data section offset, 3.
size_t gguf_alignment(const gguf_model_t* model);
size_t gguf_data_offset(const gguf_model_t* model);
uint32_t gguf_version(const gguf_model_t* model);

// Replace src/gguf_mmap.h:55 and :64: general.architecture ("" when absent); "<arch>.block_count" (0 when absent).
const char* gguf_arch(const gguf_model_t* model);
int64_t gguf_block_count(const gguf_model_t* model);

// Replace src/gguf_mmap.h:68-69: the integer (any integer or bool type) or float value of "<arch>.<suffix>", def
// when absent or an array.
int64_t gguf_arch_int(const gguf_model_t* model, const char* suffix, int64_t def);
float gguf_arch_float(const gguf_model_t* model, const char* suffix, float def);

// Replace src/gguf_mmap.h:72 and :89: a string value (NULL when not a string), the index of a key (-1: absent).
const char* gguf_kv_str_val(const gguf_model_t* model, int64_t idx);
int64_t gguf_find_kv(const gguf_model_t* model, const char* key);

// Replace src/gguf_mmap.h:81-82: a numeric array value in place in the mapping (0), -1 if absent or not numeric.
int32_t gguf_kv_get_array(const gguf_model_t* model, const char* key, int32_t* out_type, const void** out_data,
                          size_t* out_count);

// Replace src/gguf_mmap.h:96 (same as gguf_mmap_get_tensor) and :104-106 (one mapping per file of a split model).
const void* gguf_get_tensor_ptr(const gguf_model_t* model, const char* name, size_t* out_bytes);
int gguf_n_maps(const gguf_model_t* model);
const void* gguf_map_at(const gguf_model_t* model, int i, size_t* out_size);

// Replaces src/gguf_mmap.h:14-17's stderr log lines (INFER_LOG): why the last gguf_mmap_open on this thread failed.
const char* gguf_last_error(void);

#ifdef __cplusplus
}
#endif

#endif  // GGUF_MMAP_H
