/* mojotrees C ABI, served by the MI355X (gfx950) HIP library.
 *
 * Drop-in for the reference's stable C interface (ajhendel/mojoboost
 * capi/mojotrees.h, ABI version 3): the same 21 functions, the same status
 * codes and constants, the same ownership and threading rules. Each
 * declaration cites the reference line it replaces.
 *
 * What this library implements behind the ABI is the GPU training path:
 * training runs on the device (device=gpu, or device=auto when a gfx950 GPU
 * is present). A request for the CPU trainer is MOJOTREES_ERROR_UNSUPPORTED
 * with the reason, never a silent substitution. Prediction, save/load and
 * inspection run on the host.
 *
 * Rules callers may rely on (reference capi/mojotrees.h:8-34):
 *  - only C scalars, C strings, caller-owned buffers and opaque handles cross
 *    the boundary; nothing is retained after a call returns;
 *  - every fallible call returns MOJOTREES_OK or a negative error code and
 *    writes the reason into the caller's error object, cleared on entry;
 *  - every returned handle is freed by exactly one *_free call; free(NULL)
 *    is a no-op; NULL where a value is required is INVALID_ARGUMENT;
 *  - models are immutable: concurrent prediction on one model is safe with a
 *    per-thread error object and output buffer.
 */
#ifndef MOJOTREES_H
#define MOJOTREES_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference capi/mojotrees.h:84 */
#define MOJOTREES_ABI_VERSION 3

/* reference capi/mojotrees.h:86-91 */
#define MOJOTREES_OK 0
#define MOJOTREES_ERROR_INVALID_ARGUMENT (-1)
#define MOJOTREES_ERROR_TRAINING (-2)
#define MOJOTREES_ERROR_IO (-3)
#define MOJOTREES_ERROR_UNSUPPORTED (-4)

/* reference capi/mojotrees.h:101-103 */
#define MOJOTREES_DEVICE_CPU 0
#define MOJOTREES_DEVICE_GPU 1
#define MOJOTREES_DEVICE_AUTO 2

/* reference capi/mojotrees.h:108-109 */
#define MOJOTREES_PREDICT_RESPONSE 0
#define MOJOTREES_PREDICT_RAW 1

/* reference capi/mojotrees.h:115-116 */
#define MOJOTREES_IMPORTANCE_SPLIT 0
#define MOJOTREES_IMPORTANCE_GAIN 1

typedef struct MojoTreesModel MojoTreesModel;
typedef struct MojoTreesError MojoTreesError;

/* reference capi/mojotrees.h:127 */
int32_t mojotrees_abi_version(void);

/* reference capi/mojotrees.h:130-131; any out pointer may be NULL. */
void mojotrees_library_version(int32_t *major, int32_t *minor,
                               int32_t *patch);

/* reference capi/mojotrees.h:142: 1 when a gfx950 GPU is usable. */
int32_t mojotrees_gpu_available(void);

/* reference capi/mojotrees.h:147-160 */
MojoTreesError *mojotrees_error_create(void);
void mojotrees_error_free(MojoTreesError *error);
const char *mojotrees_error_message(const MojoTreesError *error);

/* reference capi/mojotrees.h:180-184. Column-major doubles
 * data[f * n_rows + r], NaN = missing; labels n_rows doubles; weights NULL
 * (unweighted) or n_rows finite, nonnegative doubles with a positive sum,
 * which scale each row's gradient and hessian and weight the base score and
 * class priors; `parameters` is a whitespace-separated LightGBM key=value
 * string. `out_model` is written only on success. */
int32_t mojotrees_train_dense(const double *data, int64_t n_rows,
                              int64_t n_features, const double *labels,
                              const double *weights, const char *parameters,
                              MojoTreesModel **out_model,
                              MojoTreesError *error);

/* reference capi/mojotrees.h:194-197: response-scale, row-major
 * out_values[r * k + c] with k = mojotrees_model_num_classes(model). */
int32_t mojotrees_predict(const MojoTreesModel *model, const double *data,
                          int64_t n_rows, int64_t n_features,
                          double *out_values, int64_t out_len,
                          MojoTreesError *error);

/* reference capi/mojotrees.h:203-206 */
int32_t mojotrees_predict_raw(const MojoTreesModel *model,
                              const double *data, int64_t n_rows,
                              int64_t n_features, double *out_values,
                              int64_t out_len, MojoTreesError *error);

/* reference capi/mojotrees.h:227-232 */
int32_t mojotrees_predict_ex(const MojoTreesModel *model, const double *data,
                             int64_t n_rows, int64_t n_features,
                             int64_t start_iteration, int64_t num_iteration,
                             int32_t flags, int32_t device,
                             double *out_values, int64_t out_len,
                             MojoTreesError *error);

/* reference capi/mojotrees.h:237-244 */
int32_t mojotrees_save_model(const MojoTreesModel *model, const char *path,
                             MojoTreesError *error);
int32_t mojotrees_load_model(const char *path, MojoTreesModel **out_model,
                             MojoTreesError *error);

/* reference capi/mojotrees.h:249-275 */
int32_t mojotrees_model_num_features(const MojoTreesModel *model,
                                     int64_t *out_value,
                                     MojoTreesError *error);
int32_t mojotrees_model_num_classes(const MojoTreesModel *model,
                                    int64_t *out_value,
                                    MojoTreesError *error);
int32_t mojotrees_model_num_trees(const MojoTreesModel *model,
                                  int64_t *out_value,
                                  MojoTreesError *error);
int32_t mojotrees_model_num_iterations(const MojoTreesModel *model,
                                       int64_t *out_value,
                                       MojoTreesError *error);

/* reference capi/mojotrees.h:289-290; release with mojotrees_string_free. */
int32_t mojotrees_model_dump_json(const MojoTreesModel *model,
                                  char **out_text, MojoTreesError *error);

/* reference capi/mojotrees.h:310-313 */
int32_t mojotrees_feature_importance(const MojoTreesModel *model,
                                     int32_t importance_type,
                                     double *out_values, int64_t out_len,
                                     MojoTreesError *error);

/* reference capi/mojotrees.h:326 */
int32_t mojotrees_parameter_keys(char **out_text, MojoTreesError *error);

/* reference capi/mojotrees.h:333-338 */
void mojotrees_string_free(char *text);
void mojotrees_model_free(MojoTreesModel *model);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* MOJOTREES_H */
