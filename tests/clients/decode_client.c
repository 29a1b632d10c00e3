/*
 * A C17 caller of the decoder surface, compiled against include/ and linked with libctorch_amd.so as a client of
 * the reference's C API would be.
 *
 * 1. The decoder block of the reference's tests/c_api.c:28-42, unchanged except for the device: this library
 *    computes on the GPU only, so the options name DL_CUDA.  A 1-layer decoder (8 features, 4 query and 2 KV
 *    heads, hidden 12, context 16) decodes a [1, 2, 8] block of ones through a cache of length 2, then clears it.
 * 2. The greedy loop of the reference's examples/decoder_generate.cpp:16-31 written against the C surface: the
 *    byte decoder of examples/decoder_model.h (vocabulary 256, 64 features, 2 layers, 4 query and 2 KV heads,
 *    hidden 256, context 128, output layer tied to the embedding) loaded from a .ct archive, the prefix decoded
 *    whole and then one byte per step, each the argmax of the last position.  Prints one id per line.
 *
 * usage: decode_client_c [<weights.ct> <prefix> [tokens]]
 */
#include <dl/c_api.h>
#include <dl/decoder_c_api.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define OK(call) do { if ((call) != DL_OK) { fprintf(stderr, "%s\n", dl_last_error()); return 1; } } while (0)

static int reference_block(void) {
    dl_tensor_options options = dl_default_tensor_options();
    options.device.type = DL_CUDA;
    dl_module* decoder;
    dl_decoder_cache* cache;
    dl_tensor *input, *square;
    OK(dl_transformer_decoder_create(1, 8, 4, 2, 12, 16, options, &decoder));
    OK(dl_decoder_cache_create(decoder, &cache));
    const int64_t sequence_dims[] = {1, 2, 8};
    OK(dl_ones((dl_shape){sequence_dims, 3}, options, &input));
    OK(dl_transformer_decoder_decode(decoder, input, cache, &square));
    int64_t length;
    OK(dl_decoder_cache_length(cache, &length));
    if (length != 2) return 1;
    OK(dl_decoder_cache_clear(cache));
    float values[16];
    OK(dl_tensor_copy_to_host(square, values));
    for (int i = 0; i < 16; ++i)
        if (values[i] != values[i]) return 1; /* NaN */
    dl_tensor_release(square);
    dl_tensor_release(input);
    dl_decoder_cache_release(cache);
    dl_module_release(decoder);
    printf("reference block: cache length 2\n");
    return 0;
}

static const char* state_find(const dl_state* state, const char* name, size_t* index) {
    for (size_t i = 0; i < dl_state_size(state); ++i)
        if (strcmp(dl_state_name(state, i), name) == 0) {
            *index = i;
            return dl_state_name(state, i);
        }
    return NULL;
}

static int generate(const char* path, const char* prefix, int64_t count) {
    const dl_device gpu = {DL_CUDA, 0};
    dl_state* state;
    OK(dl_state_load(path, &state));
    size_t at;
    dl_tensor *host, *tokens, *head;
    if (!state_find(state, "tokens.weight", &at) || !state_find(state, "output.weight", &at)) return 1;
    state_find(state, "tokens.weight", &at);
    OK(dl_state_tensor(state, at, &host));
    OK(dl_to(host, gpu, &tokens));
    dl_tensor_release(host);
    state_find(state, "output.weight", &at);
    OK(dl_state_tensor(state, at, &host));
    OK(dl_to(host, gpu, &head));
    dl_tensor_release(host);
    dl_module *embedding, *output, *decoder;
    OK(dl_embedding_from_tensor(tokens, &embedding));
    OK(dl_linear_from_tensors(head, NULL, &output));
    dl_tensor_options options = dl_default_tensor_options();
    options.device = gpu;
    OK(dl_transformer_decoder_create(2, 64, 4, 2, 256, 128, options, &decoder));

    /* the decoder's entries, named relative to the decoder */
    const size_t total = dl_state_size(state);
    const char** names = calloc(total, sizeof(char*));
    dl_tensor** tensors = calloc(total, sizeof(dl_tensor*));
    size_t n = 0;
    for (size_t i = 0; i < total; ++i) {
        const char* name = dl_state_name(state, i);
        if (strncmp(name, "decoder.", 8) != 0) continue;
        names[n] = name + 8;
        OK(dl_state_tensor(state, i, &tensors[n]));
        ++n;
    }
    dl_state* decoder_state;
    OK(dl_state_create(names, (const dl_tensor* const*)tensors, n, &decoder_state));
    OK(dl_module_load_state(decoder, decoder_state));
    dl_state_release(decoder_state);
    for (size_t i = 0; i < n; ++i) dl_tensor_release(tensors[i]);
    free(tensors);
    free(names);
    dl_state_release(state);

    dl_decoder_cache* cache;
    OK(dl_decoder_cache_create(decoder, &cache));
    const int64_t length = (int64_t)strlen(prefix);
    if (length == 0 || count < 0 || length + count > 128) return 1;
    int64_t ids[128];
    for (int64_t i = 0; i < length; ++i) ids[i] = (unsigned char)prefix[i];
    const dl_tensor_options indices = {DL_I64, gpu, 0};
    const int64_t dims[] = {1, length};
    dl_tensor* input;
    OK(dl_from_host(ids, (dl_shape){dims, 2}, indices, &input));
    for (int64_t i = 0; i < count; ++i) {
        dl_tensor *embedded, *hidden, *last, *logits, *next;
        OK(dl_module_forward(embedding, input, &embedded));
        OK(dl_transformer_decoder_decode(decoder, embedded, cache, &hidden));
        const int64_t positions = dl_tensor_shape(input).data[1];
        OK(dl_select(hidden, 1, positions - 1, &last));
        OK(dl_module_forward(output, last, &logits));
        OK(dl_argmax(logits, -1, 0, &next));
        int64_t id;
        OK(dl_tensor_copy_to_host(next, &id));
        printf("%lld\n", (long long)id);
        dl_tensor_release(next);
        dl_tensor_release(logits);
        dl_tensor_release(last);
        dl_tensor_release(hidden);
        dl_tensor_release(embedded);
        dl_tensor_release(input);
        const int64_t one[] = {1, 1};
        OK(dl_full((dl_shape){one, 2}, (double)id, indices, &input));
    }
    dl_tensor_release(input);
    dl_decoder_cache_release(cache);
    dl_module_release(decoder);
    dl_module_release(output);
    dl_module_release(embedding);
    dl_tensor_release(head);
    dl_tensor_release(tokens);
    return 0;
}

int main(int argc, char** argv) {
    if (reference_block()) return 1;
    if (argc < 3) return 0;
    return generate(argv[1], argv[2], argc > 3 ? atoll(argv[3]) : 32);
}
