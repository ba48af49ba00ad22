/*
 * Prints the ABI facts of the public header it is compiled against: sizes
 * and field offsets of every struct, and every enum value. Compiled once
 * against include/slipstream.h and once against the reference's
 * SlipStream/include/slipstream.h; the two outputs must agree on every
 * line the reference's header defines. Test infrastructure.
 */
#include <stddef.h>
#include <stdio.h>

#include "slipstream.h"

#define SZ(t) printf("sizeof %s %zu\n", #t, sizeof(t))
#define OFF(t, f) printf("offsetof %s.%s %zu\n", #t, #f, offsetof(t, f))
#define VAL(e) printf("value %s %d\n", #e, (int)(e))

int main(void) {
    SZ(ss_model_info_t);
    OFF(ss_model_info_t, model_name); OFF(ss_model_info_t, architecture); OFF(ss_model_info_t, chat_format);
    OFF(ss_model_info_t, num_layers); OFF(ss_model_info_t, hidden_size); OFF(ss_model_info_t, num_heads);
    OFF(ss_model_info_t, num_kv_heads); OFF(ss_model_info_t, vocab_size); OFF(ss_model_info_t, context_length);
    OFF(ss_model_info_t, intermediate_size); OFF(ss_model_info_t, quant_type); OFF(ss_model_info_t, file_size);
    OFF(ss_model_info_t, per_layer_size);
    SZ(ss_model_config_t);
    OFF(ss_model_config_t, backend); OFF(ss_model_config_t, n_threads); OFF(ss_model_config_t, max_memory);
    OFF(ss_model_config_t, use_mmap); OFF(ss_model_config_t, prefetch); OFF(ss_model_config_t, context_size);
    SZ(ss_generate_params_t);
    OFF(ss_generate_params_t, max_tokens); OFF(ss_generate_params_t, temperature); OFF(ss_generate_params_t, top_p);
    OFF(ss_generate_params_t, top_k); OFF(ss_generate_params_t, repeat_penalty); OFF(ss_generate_params_t, seed);
    OFF(ss_generate_params_t, stop_sequence);
    SZ(ss_device_info_t);
    OFF(ss_device_info_t, device_model); OFF(ss_device_info_t, chip_name); OFF(ss_device_info_t, cpu_core_count);
    OFF(ss_device_info_t, perf_core_count); OFF(ss_device_info_t, efficiency_core_count);
    OFF(ss_device_info_t, gpu_core_count); OFF(ss_device_info_t, total_memory);
    OFF(ss_device_info_t, available_memory); OFF(ss_device_info_t, thermal_state);
    SZ(ss_error_t); SZ(ss_backend_t); SZ(ss_quant_type_t);
    VAL(SS_OK); VAL(SS_ERROR_FILE_NOT_FOUND); VAL(SS_ERROR_INVALID_MODEL); VAL(SS_ERROR_OUT_OF_MEMORY);
    VAL(SS_ERROR_MMAP_FAILED); VAL(SS_ERROR_INVALID_PARAMS); VAL(SS_ERROR_CANCELLED); VAL(SS_ERROR_BACKEND);
    VAL(SS_ERROR_TOKENIZER); VAL(SS_ERROR_UNKNOWN);
    VAL(SS_BACKEND_AUTO); VAL(SS_BACKEND_CPU); VAL(SS_BACKEND_METAL);
    VAL(SS_QUANT_F32); VAL(SS_QUANT_F16); VAL(SS_QUANT_Q8_0); VAL(SS_QUANT_Q4_0); VAL(SS_QUANT_Q4_1);
    VAL(SS_VERSION_MAJOR); VAL(SS_VERSION_MINOR); VAL(SS_VERSION_PATCH);
    printf("string SS_VERSION_STRING %s\n", SS_VERSION_STRING);
    return 0;
}
