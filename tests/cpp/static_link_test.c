/* Links libqlinear.a the way the reference's build.rs links its native library
 * (build.rs:13-67: a static archive pulled in whole, plus the runtime it needs) and
 * calls entry points that reject their arguments before any device work, so it runs
 * on a host without a GPU. */
#include <stdio.h>
#include <string.h>

#include "../../include/qlinear.h"

int main(void) {
    if (strcmp(qlin_strerror(QLIN_OK), "success") != 0) return 1;
    if (strcmp(qlin_strerror(QLIN_ERR_PARAM), "invalid parameter") != 0) return 2;
    if (strcmp(qlin_strerror(-99), "unknown error") != 0) return 3;
    qlin_weights* w = (qlin_weights*)&w;
    if (qlin_weights_create(NULL, NULL, NULL, &w) != QLIN_ERR_PARAM || w != NULL) return 4;
    qlin_weight_config bad_bits = {3, 8, 8};
    int8_t codes[64] = {0};
    float scales[8] = {1, 1, 1, 1, 1, 1, 1, 1};
    if (qlin_weights_create(&bad_bits, codes, scales, &w) != QLIN_ERR_PARAM || w != NULL) return 5;
    qlin_weight_config cfg = {4, 8, 8};
    codes[9] = 8; /* outside W4 [-8, 7] */
    if (qlin_weights_create(&cfg, codes, scales, &w) != QLIN_ERR_PARAM || w != NULL) return 6;
    codes[9] = 0;
    scales[3] = 0.0f; /* scales must be positive */
    if (qlin_weights_create(&cfg, codes, scales, &w) != QLIN_ERR_PARAM || w != NULL) return 7;
    if (qlin_run(NULL, NULL, 1, NULL, QLIN_F16, 8, NULL, QLIN_F16, 8, 0, NULL) != QLIN_ERR_PARAM) return 8;
    if (qlin_run_f32(NULL, NULL, 1, NULL, NULL) != QLIN_ERR_PARAM) return 9;
    qlin_weights_free(NULL);
    qlin_workspace_free(NULL);
    printf("static link ok\n");
    return 0;
}
