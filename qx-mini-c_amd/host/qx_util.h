/* Helpers shared by the host probe files (not part of the public API). */
#ifndef QX_UTIL_H
#define QX_UTIL_H

#include "qx_host.h"
#include "qxg.h"

#include <stdint.h>
#include <stdio.h>

void qxh_set_err(char *err, uint64_t n, const char *msg);
/* the reference's exact-size F32 sidecar read (src/qx_format.c:5319-5344): the file holds
 * exactly n finite floats */
int qxh_read_sidecar(const char *path, float *v, uint32_t n, char *err, uint64_t err_len);
/* dir/name.f32 with n floats; a partial file is removed */
int qxh_write_f32(const char *dir, const char *name, const float *v, uint64_t n, char *err, uint64_t err_len);
void qxh_remove_f32(const char *dir, const char *name);
/* "f32" -> 0, "q8_k_compat" -> 1, anything else -> -1 */
int qxh_activation_code(const char *s);
/* device 0, the file's tensors uploaded and bound (checksums verified when verify) */
int qxh_open_gpu(const char *path, int verify, qxg_ctx **ctx, qx_gpu_model_info *mi, char *err, uint64_t err_len);
double qxh_now_s(void);
/* the reference's projection kernel labels (src/qx_format.c:4347-4373) */
uint32_t qxh_projection_family_bit(uint32_t ggml_type);
const char *qxh_projection_kernel_label(uint32_t family_mask, int f32_used);
const char *qxh_projection_tensor_kernel_label(uint32_t ggml_type, int use_q8_k);
/* blk.<layer>.<suffix> in the file's directory, or NULL */
const qxf_dir_entry *qxh_layer_tensor(const qxf_file *f, uint32_t layer, const char *suffix);
/* JSON string with the reference's escaping (qx_json_print_escaped) */
void qxh_json_string(FILE *out, const char *s);

#endif
