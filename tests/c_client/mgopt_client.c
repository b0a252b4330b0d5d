/* A C caller of libmgopt: the optimizer step of train.py:483-491 driven
 * through include/mgopt.h alone, compiled as C99 and linked against the
 * library and the HIP runtime, with no Python or torch in the process.
 *
 * Three tensors in two groups: 5,000 fp32 parameters with fp32 gradients,
 * 70,000 bf16 parameters with an fp32 master and bf16 gradients, 129 fp32
 * parameters with fp16 gradients.  Parameters and gradients come from the
 * library's deterministic generator (mgopt_synth_fill), for which the test
 * oracle has a bit-identical host twin.  Six steps of unscale + norm + clip
 * (1.0) + AdamW + scaler update (initial scale 1,024, growth interval 2); at
 * step 4 the last gradient element of the third tensor is a NaN, so that
 * step is skipped.
 *
 * Usage: mgopt_client OUT_FILE.  Writes, in this order, as raw little-endian
 * data: per step the norm (float), found_inf (float), scale after the update
 * (float) and growth tracker (int32); then per tensor its fp32 values (the
 * master for the bf16 tensor), exp_avg, exp_avg_sq and, for the bf16 tensor,
 * its parameter bits; then the three step counts (float).  Exit status 0 on
 * success. */

#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "mgopt.h"

#define N_TENSORS 3
#define N_STEPS 6
#define BC_CAP 64

static int check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
        return 1;
    }
    return 0;
}

static int check_mg(int rc, const char* what) {
    if (rc != 0) {
        fprintf(stderr, "%s: rc %d: %s\n", what, rc, mgopt_last_error());
        return 1;
    }
    return 0;
}

/* the generator's multiplier for standard deviation sigma (Irwin-Hall of four
 * 16-bit uniforms) */
static double synth_k(double sigma) { return sigma * sqrt(3.0) / 65536.0; }

static int elem_size(int32_t dtype) { return dtype == MGOPT_F32 ? 4 : 2; }

int main(int argc, char** argv) {
    if (argc != 2) {
        fprintf(stderr, "usage: %s OUT_FILE\n", argv[0]);
        return 2;
    }
    const int64_t numel[N_TENSORS] = {5000, 70000, 129};
    const int32_t param_dtype[N_TENSORS] = {MGOPT_F32, MGOPT_BF16, MGOPT_F32};
    const int32_t grad_dtype[N_TENSORS] = {MGOPT_F32, MGOPT_BF16, MGOPT_F16};
    const int32_t group[N_TENSORS] = {0, 0, 1};
    const double weight_decay[2] = {0.1, 0.0};
    const double beta1 = 0.9, beta2 = 0.95, eps = 1e-8;

    void* param[N_TENSORS];
    void* grad[N_TENSORS];
    float* master[N_TENSORS];
    float* m[N_TENSORS];
    float* v[N_TENSORS];
    float *steps, *scale, *norm, *coef, *found;
    int32_t* tracker;
    double* bc;
    mgopt_tensor_desc descs[N_TENSORS];
    memset(descs, 0, sizeof(descs));

    for (int i = 0; i < N_TENSORS; ++i) {
        const size_t n = (size_t)numel[i];
        if (check_hip(hipMalloc(&param[i], n * elem_size(param_dtype[i])), "hipMalloc param") ||
            check_hip(hipMalloc(&grad[i], n * elem_size(grad_dtype[i])), "hipMalloc grad") ||
            check_hip(hipMalloc((void**)&m[i], n * 4), "hipMalloc exp_avg") ||
            check_hip(hipMalloc((void**)&v[i], n * 4), "hipMalloc exp_avg_sq") ||
            check_hip(hipMemset(m[i], 0, n * 4), "clear exp_avg") || check_hip(hipMemset(v[i], 0, n * 4), "clear exp_avg_sq"))
            return 1;
        master[i] = NULL;
        if (param_dtype[i] != MGOPT_F32 && check_hip(hipMalloc((void**)&master[i], n * 4), "hipMalloc master")) return 1;
        if (check_mg(mgopt_synth_fill(param[i], param_dtype[i], numel[i], 1, (uint64_t)i, synth_k(0.02), 0, 1.0, NULL),
                     "synth params"))
            return 1;
        descs[i].param_dev = master[i] ? master[i] : (float*)param[i];
        descs[i].lowp_dev = master[i] ? param[i] : NULL;
        descs[i].lowp_dtype = master[i] ? param_dtype[i] : MGOPT_NONE;
        descs[i].exp_avg_dev = m[i];
        descs[i].exp_avg_sq_dev = v[i];
        descs[i].numel = numel[i];
        descs[i].group = group[i];
        descs[i].grad_dtype = grad_dtype[i];
    }
    if (check_hip(hipMalloc((void**)&steps, N_TENSORS * 4), "hipMalloc steps") ||
        check_hip(hipMemset(steps, 0, N_TENSORS * 4), "clear steps") ||
        check_hip(hipMalloc((void**)&scale, 4), "hipMalloc scale") ||
        check_hip(hipMalloc((void**)&tracker, 4), "hipMalloc tracker") ||
        check_hip(hipMalloc((void**)&norm, 4), "hipMalloc norm") || check_hip(hipMalloc((void**)&coef, 4), "hipMalloc coef") ||
        check_hip(hipMalloc((void**)&found, 4), "hipMalloc found"))
        return 1;
    const float scale0 = 1024.0f;
    const int32_t tracker0 = 0;
    if (check_hip(hipMemcpy(scale, &scale0, 4, hipMemcpyHostToDevice), "scale") ||
        check_hip(hipMemcpy(tracker, &tracker0, 4, hipMemcpyHostToDevice), "tracker"))
        return 1;

    /* bias corrections as torch/optim/adam.py:529-536 forms them, with each
     * group's betas at t = 0 */
    double host_bc[2 * BC_CAP * 2];
    for (int g = 0; g < 2; ++g) {
        host_bc[(g * BC_CAP) * 2] = beta1;
        host_bc[(g * BC_CAP) * 2 + 1] = beta2;
        for (int t = 1; t < BC_CAP; ++t) {
            host_bc[(g * BC_CAP + t) * 2] = 1.0 - pow(beta1, (double)t);
            host_bc[(g * BC_CAP + t) * 2 + 1] = pow(1.0 - pow(beta2, (double)t), 0.5);   /* Python's ** 0.5 */
        }
    }
    if (check_hip(hipMalloc((void**)&bc, sizeof(host_bc)), "hipMalloc bc") ||
        check_hip(hipMemcpy(bc, host_bc, sizeof(host_bc), hipMemcpyHostToDevice), "bc"))
        return 1;

    mgopt_plan* plan = NULL;
    if (check_mg(mgopt_plan_create(descs, N_TENSORS, 2, steps, 65536, &plan), "plan_create")) return 1;
    if (check_mg(mgopt_sync_master(plan, NULL), "sync_master")) return 1;

    FILE* out = fopen(argv[1], "wb");
    if (!out) {
        perror("fopen");
        return 1;
    }
    mgopt_group_hparams hp[2];
    memset(hp, 0, sizeof(hp));
    for (int g = 0; g < 2; ++g) {
        hp[g].weight_decay = weight_decay[g];
        hp[g].beta1 = beta1;
        hp[g].beta2 = beta2;
        hp[g].eps = eps;
    }
    const void* grads_host[N_TENSORS] = {grad[0], grad[1], grad[2]};
    const float* found_list[1] = {found};
    float cur_scale = scale0;
    for (int s = 1; s <= N_STEPS; ++s) {
        const double lr = 1e-3 * (0.5 + 0.1 * s);
        hp[0].lr = hp[1].lr = lr;
        for (int i = 0; i < N_TENSORS; ++i)
            if (check_mg(mgopt_synth_fill(grad[i], grad_dtype[i], numel[i], 2, ((uint64_t)s << 20) | (uint64_t)i,
                                          synth_k(1e-2 * cur_scale), 0, 1.0, NULL),
                         "synth grads"))
                return 1;
        if (s == 4) {
            const uint16_t half_nan = 0x7E00u;
            if (check_hip(hipMemcpy((uint16_t*)grad[2] + numel[2] - 1, &half_nan, 2, hipMemcpyHostToDevice), "nan"))
                return 1;
        }
        if (check_mg(mgopt_plan_set_grads(plan, grads_host, NULL), "set_grads") ||
            check_mg(mgopt_grad_norm(plan, scale, 1.0, norm, coef, found, NULL), "grad_norm") ||
            check_mg(mgopt_adamw_step(plan, hp, bc, BC_CAP, scale, coef, found, 0, NULL), "adamw_step") ||
            check_mg(mgopt_scaler_update(scale, tracker, found_list, 1, 2.0, 0.5, 2, NULL), "scaler_update"))
            return 1;
        float rec[3];
        int32_t trk;
        if (check_hip(hipMemcpy(&rec[0], norm, 4, hipMemcpyDeviceToHost), "read norm") ||
            check_hip(hipMemcpy(&rec[1], found, 4, hipMemcpyDeviceToHost), "read found") ||
            check_hip(hipMemcpy(&rec[2], scale, 4, hipMemcpyDeviceToHost), "read scale") ||
            check_hip(hipMemcpy(&trk, tracker, 4, hipMemcpyDeviceToHost), "read tracker"))
            return 1;
        cur_scale = rec[2];
        fwrite(rec, 4, 3, out);
        fwrite(&trk, 4, 1, out);
    }
    for (int i = 0; i < N_TENSORS; ++i) {
        const size_t n = (size_t)numel[i];
        float* host = (float*)malloc(n * 4);
        uint16_t* bits = (uint16_t*)malloc(n * 2);
        if (!host || !bits) return 1;
        const float* arrays[3] = {master[i] ? master[i] : (const float*)param[i], m[i], v[i]};
        for (int k = 0; k < 3; ++k) {
            if (check_hip(hipMemcpy(host, arrays[k], n * 4, hipMemcpyDeviceToHost), "read state")) return 1;
            fwrite(host, 4, n, out);
        }
        if (master[i]) {
            if (check_hip(hipMemcpy(bits, param[i], n * 2, hipMemcpyDeviceToHost), "read bf16")) return 1;
            fwrite(bits, 2, n, out);
        }
        free(host);
        free(bits);
    }
    float host_steps[N_TENSORS];
    if (check_hip(hipMemcpy(host_steps, steps, sizeof(host_steps), hipMemcpyDeviceToHost), "read steps")) return 1;
    fwrite(host_steps, 4, N_TENSORS, out);
    fclose(out);
    mgopt_plan_destroy(plan);
    printf("mgopt_client: %d steps, %s\n", N_STEPS, mgopt_version());
    return 0;
}
