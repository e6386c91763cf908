/* A C99 program against include/mojotrees.h that calls every one of its 21
 * functions through the shared library, with no GPU: the reference's
 * capi/test_capi.c checks the same calls. argv[1] is a scratch directory.
 * Exits 0 and prints "ok" when every check holds. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "mojotrees.h"

static int failures = 0;
#define CHECK(cond)                                                     \
    do {                                                                \
        if (!(cond)) {                                                  \
            fprintf(stderr, "check failed at line %d: %s\n", __LINE__, #cond); \
            ++failures;                                                 \
        }                                                               \
    } while (0)

static void write_bits(FILE *f, double x) {
    uint64_t u;
    memcpy(&u, &x, sizeof u);
    fprintf(f, "%llu", (unsigned long long)u);
}

int main(int argc, char **argv) {
    if (argc < 2) return 2;
    char path[4096], path2[4096];
    snprintf(path, sizeof path, "%s/v1.txt", argv[1]);
    snprintf(path2, sizeof path2, "%s/v4.txt", argv[1]);

    CHECK(mojotrees_abi_version() == MOJOTREES_ABI_VERSION);
    int32_t major = -1, minor = -1, patch = -1;
    mojotrees_library_version(&major, &minor, &patch);
    CHECK(major >= 0 && minor >= 0 && patch >= 0);
    mojotrees_library_version(NULL, NULL, NULL);
    const int32_t gpu = mojotrees_gpu_available();
    CHECK(gpu == 0 || gpu == 1);

    MojoTreesError *err = mojotrees_error_create();
    CHECK(err != NULL);
    CHECK(mojotrees_error_message(err) != NULL);

    /* device=cpu is not served: UNSUPPORTED, out_model untouched */
    double data[8] = {1, 2, 3, 4, 5, 6, 7, 8}, labels[4] = {0, 1, 0, 1};
    MojoTreesModel *trained = NULL;
    CHECK(mojotrees_train_dense(data, 4, 2, labels, NULL, "objective=binary device=cpu", &trained, err) ==
          MOJOTREES_ERROR_UNSUPPORTED);
    CHECK(trained == NULL);
    CHECK(strlen(mojotrees_error_message(err)) > 0);
    CHECK(mojotrees_train_dense(data, 4, 2, labels, NULL, "no_such_key=1", &trained, err) ==
          MOJOTREES_ERROR_INVALID_ARGUMENT);

    /* the reference's v1 model file (tests/test_serialize.mojo:246-270) */
    FILE *f = fopen(path, "w");
    CHECK(f != NULL);
    if (!f) return 1;
    fprintf(f, "mojotrees v1\nobjective 0\nlearning_rate ");
    write_bits(f, 0.5);
    fprintf(f, "\nbase_score ");
    write_bits(f, 1.0);
    fprintf(f, "\nmapper 1 4 1\n");
    write_bits(f, 2.0);
    fprintf(f, "\n0 1\ntrees 1\ntree 3 2\n0 -1 -1\n0 -1 -1\n1 -1 -1\n2 -1 -1\n");
    write_bits(f, 0.0);
    fputc(' ', f);
    write_bits(f, 10.0);
    fputc(' ', f);
    write_bits(f, 20.0);
    fputc('\n', f);
    fclose(f);

    MojoTreesModel *model = NULL;
    CHECK(mojotrees_load_model(path, &model, err) == MOJOTREES_OK);
    if (!model) {
        fprintf(stderr, "load failed: %s\n", mojotrees_error_message(err));
        return 1;
    }
    int64_t v = 0;
    CHECK(mojotrees_model_num_features(model, &v, err) == MOJOTREES_OK && v == 1);
    CHECK(mojotrees_model_num_classes(model, &v, err) == MOJOTREES_OK && v == 1);
    CHECK(mojotrees_model_num_trees(model, &v, err) == MOJOTREES_OK && v == 1);
    CHECK(mojotrees_model_num_iterations(model, &v, err) == MOJOTREES_OK && v == 1);

    double x[2] = {1.0, 3.0}, out[2] = {0, 0};
    CHECK(mojotrees_predict(model, x, 2, 1, out, 2, err) == MOJOTREES_OK);
    CHECK(out[0] == 1.0 + 0.5 * 10.0 && out[1] == 1.0 + 0.5 * 20.0);
    CHECK(mojotrees_predict_raw(model, x, 2, 1, out, 2, err) == MOJOTREES_OK);
    CHECK(out[0] == 6.0 && out[1] == 11.0);
    CHECK(mojotrees_predict_ex(model, x, 2, 1, 0, 0, MOJOTREES_PREDICT_RAW, MOJOTREES_DEVICE_CPU, out, 2,
                               err) == MOJOTREES_OK);
    CHECK(out[0] == 6.0 && out[1] == 11.0);
    CHECK(mojotrees_predict(model, x, 2, 1, out, 1, err) == MOJOTREES_ERROR_INVALID_ARGUMENT);

    CHECK(mojotrees_save_model(model, path2, err) == MOJOTREES_OK);
    MojoTreesModel *again = NULL;
    CHECK(mojotrees_load_model(path2, &again, err) == MOJOTREES_OK);
    if (again) {
        CHECK(mojotrees_predict(again, x, 2, 1, out, 2, err) == MOJOTREES_OK);
        CHECK(out[0] == 6.0 && out[1] == 11.0);
    }

    char *text = NULL;
    CHECK(mojotrees_model_dump_json(model, &text, err) == MOJOTREES_OK && text != NULL);
    if (text) CHECK(strstr(text, "\"num_trees\":1") != NULL);
    mojotrees_string_free(text);

    double imp[1] = {-1.0};
    CHECK(mojotrees_feature_importance(model, MOJOTREES_IMPORTANCE_SPLIT, imp, 1, err) == MOJOTREES_OK);
    CHECK(imp[0] == 1.0);

    char *keys = NULL;
    CHECK(mojotrees_parameter_keys(&keys, err) == MOJOTREES_OK && keys != NULL);
    if (keys) CHECK(strstr(keys, "num_leaves") != NULL);
    mojotrees_string_free(keys);
    mojotrees_string_free(NULL);

    mojotrees_model_free(again);
    mojotrees_model_free(model);
    mojotrees_model_free(NULL);
    mojotrees_error_free(err);
    mojotrees_error_free(NULL);
    if (failures) return 1;
    printf("ok\n");
    return 0;
}
