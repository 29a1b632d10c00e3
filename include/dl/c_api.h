#ifndef CTORCH_C_API_H
#define CTORCH_C_API_H
/*
 * C17 surface of the decoder token loop.  Every declaration keeps the name, argument order and meaning of
 * the reference's include/dl/c_api.h (line numbers cited per group) so that a C caller of the reference
 * relinks against this library unchanged.  Only the subset on the decode path is provided.
 *
 * Conventions (reference c_api.h:154-158): entries that create or compute return a new owned handle through
 * an output slot that is set to NULL on failure; status entries return DL_ERROR and keep the failure text
 * for the calling thread (dl_last_error); *_release accepts NULL.
 *
 * Device naming: the reference's spellings are kept so that its C callers compile unchanged.  DL_CUDA (value 1)
 * names the HIP GPU in this library, DL_GPU is an alias, and the pool statistics keep their dl_cuda_memory_*
 * names (dl_gpu_memory_* are aliases).
 */
#include "dl/export.h"

#include <stddef.h>
#include <stdint.h>
#include <stdbool.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct dl_tensor dl_tensor;
typedef struct dl_module dl_module;
typedef struct dl_state dl_state;

/* c_api.h:34-36,43,51,54-58,89 */
typedef enum dl_status { DL_OK = 0, DL_ERROR = 1 } dl_status;
typedef enum dl_dtype { DL_F32 = 0, DL_F64 = 1, DL_I64 = 2, DL_BOOL = 3, DL_F16 = 4, DL_BF16 = 5 } dl_dtype;
typedef enum dl_device_type { DL_CPU = 0, DL_CUDA = 1, DL_GPU = DL_CUDA } dl_device_type;
typedef struct dl_device { dl_device_type type; int32_t index; } dl_device;
typedef struct dl_shape { const int64_t* data; size_t size; } dl_shape;
typedef struct dl_tensor_options {
    dl_dtype dtype;
    dl_device device;
    int32_t requires_grad;
} dl_tensor_options;
typedef struct dl_tensor_info {
    dl_dtype dtype;
    dl_device device;
    int64_t numel;
    int32_t contiguous, requires_grad, leaf;
} dl_tensor_info;
typedef struct dl_random_key { uint64_t seed, stream; } dl_random_key;
/* Pool statistics of this library's device allocator (reference c_api.h:46-50). */
typedef struct dl_cuda_memory_stats {
    uint64_t used_bytes, reserved_bytes;
    uint64_t peak_used_bytes, peak_reserved_bytes;
    uint64_t release_threshold;
} dl_cuda_memory_stats;
typedef dl_cuda_memory_stats dl_gpu_memory_stats;

/* c_api.h:159-161 */
DL_API const char* dl_version(void);
DL_API const char* dl_last_error(void);
DL_API dl_tensor_options dl_default_tensor_options(void);

/* c_api.h:177-191: handles, metadata and host round trips */
DL_API void dl_tensor_release(dl_tensor* tensor);
DL_API dl_status dl_tensor_retain(const dl_tensor* tensor, dl_tensor** output);
DL_API dl_tensor_info dl_tensor_get_info(const dl_tensor* tensor);
DL_API dl_shape dl_tensor_shape(const dl_tensor* tensor);
DL_API dl_shape dl_tensor_strides(const dl_tensor* tensor);
DL_API const void* dl_tensor_data(const dl_tensor* tensor);
DL_API size_t dl_tensor_nbytes(const dl_tensor* tensor);
DL_API dl_status dl_tensor_copy_to_host(const dl_tensor* tensor, void* destination);
DL_API dl_status dl_from_host(const void* data, dl_shape shape, dl_tensor_options options, dl_tensor** output);
DL_API dl_status dl_full(dl_shape shape, double value, dl_tensor_options options, dl_tensor** output);
DL_API dl_status dl_zeros(dl_shape shape, dl_tensor_options options, dl_tensor** output);
DL_API dl_status dl_ones(dl_shape shape, dl_tensor_options options, dl_tensor** output);

/* c_api.h:200-218: copies, casts, transfers and views */
DL_API dl_status dl_clone(const dl_tensor* input, dl_tensor** output);
DL_API dl_status dl_contiguous(const dl_tensor* input, dl_tensor** output);
DL_API dl_status dl_astype(const dl_tensor* input, dl_dtype dtype, dl_tensor** output);
DL_API dl_status dl_to(const dl_tensor* input, dl_device device, dl_tensor** output);
DL_API dl_status dl_reshape(const dl_tensor* input, dl_shape shape, dl_tensor** output);
DL_API dl_status dl_select(const dl_tensor* input, int64_t axis, int64_t index, dl_tensor** output);
DL_API dl_status dl_narrow(const dl_tensor* input, int64_t axis, int64_t start, int64_t length, dl_tensor** output);

/* c_api.h:283,306,313,378: decode-path operators */
DL_API dl_status dl_argmax(const dl_tensor* input, int64_t axis, int32_t keepdim, dl_tensor** output);
DL_API dl_status dl_linear(const dl_tensor* input, const dl_tensor* weight, const dl_tensor* bias,
    dl_tensor** output);
DL_API dl_status dl_embedding(const dl_tensor* indices, const dl_tensor* weight, dl_tensor** output);
DL_API dl_status dl_rms_norm(const dl_tensor* input, dl_shape normalized_shape,
    const dl_tensor* weight, const double* epsilon, dl_tensor** output);

/* c_api.h:488-499: grad mode, device synchronisation and the allocator's pool statistics */
DL_API dl_status dl_synchronize(dl_device device);
DL_API int32_t dl_grad_enabled(void);
DL_API dl_status dl_cuda_memory_get_stats(int32_t device, dl_cuda_memory_stats* output);
DL_API dl_status dl_cuda_memory_set_release_threshold(int32_t device, uint64_t bytes);
DL_API dl_status dl_cuda_memory_reset_peak_stats(int32_t device);
DL_API dl_status dl_cuda_memory_release_unused(int32_t device);
/* the same four entries under this library's device name */
DL_API dl_status dl_gpu_memory_get_stats(int32_t device, dl_gpu_memory_stats* output);
DL_API dl_status dl_gpu_memory_set_release_threshold(int32_t device, uint64_t bytes);
DL_API dl_status dl_gpu_memory_reset_peak_stats(int32_t device);
DL_API dl_status dl_gpu_memory_release_unused(int32_t device);

/* c_api.h:512-521: explicit-key randomness */
DL_API dl_random_key dl_random_fold_in(dl_random_key key, uint64_t label);
DL_API void dl_random_split(dl_random_key key, size_t count, dl_random_key* outputs);
DL_API dl_status dl_uniform_with_key(dl_random_key key, dl_shape shape, double low, double high,
    dl_tensor_options options, dl_tensor** output);
DL_API dl_status dl_randn_with_key(dl_random_key key, dl_shape shape, dl_tensor_options options, dl_tensor** output);

/* c_api.h:524-533,549: modules */
DL_API void dl_module_release(dl_module* module);
DL_API dl_status dl_module_retain(const dl_module* module, dl_module** output);
DL_API dl_status dl_linear_create(int64_t input_features, int64_t output_features, int32_t bias,
    dl_tensor_options options, dl_module** output);
DL_API dl_status dl_linear_from_tensors(const dl_tensor* weight, const dl_tensor* bias, dl_module** output);
DL_API dl_status dl_embedding_create(int64_t vocabulary, int64_t dimensions, dl_tensor_options options,
    dl_module** output);
DL_API dl_status dl_embedding_from_tensor(const dl_tensor* weight, dl_module** output);
DL_API dl_status dl_rms_norm_create(dl_shape normalized_shape, const double* epsilon, int32_t affine,
    dl_tensor_options options, dl_module** output);

/* c_api.h:619,631,637-646: forward, device moves and named state */
DL_API dl_status dl_module_forward(dl_module* module, const dl_tensor* input, dl_tensor** output);
DL_API dl_status dl_module_to(dl_module* module, dl_device device);
DL_API dl_status dl_module_parameters(const dl_module* module, dl_state** output);
DL_API dl_status dl_module_state(const dl_module* module, dl_state** output);
DL_API dl_status dl_module_load_state(dl_module* module, const dl_state* state);
DL_API void dl_state_release(dl_state* state);
DL_API size_t dl_state_size(const dl_state* state);
DL_API const char* dl_state_name(const dl_state* state, size_t index);
DL_API dl_status dl_state_tensor(const dl_state* state, size_t index, dl_tensor** output);
DL_API dl_status dl_state_create(const char* const* names, const dl_tensor* const* tensors, size_t count,
    dl_state** output);
/* c_api.h:647-648: the named state as a version-1 tensor archive (dl/io.h); load gives CPU tensors */
DL_API dl_status dl_state_save(const char* path, const dl_state* state);
DL_API dl_status dl_state_load(const char* path, dl_state** output);

#ifdef __cplusplus
}
#endif

#endif
