// Exhaustive host check of the device expf/sigmoid source (sf37_dev.h):
// every binary32 input against the host libm expf and the engine sigmoid
// (sf37_ops.c:9-16).  Built and run by tests/test_abi.py.
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "sf37_dev.h"

static float host_sigmoid(float x) {
    if (x >= 0.0f) {
        const float z = expf(-x);
        return 1.0f / (1.0f + z);
    }
    const float z = expf(x);
    return z / (1.0f + z);
}

struct job { uint64_t lo, hi, bad_exp, bad_sig; };

static void *run(void *p) {
    job *j = (job *)p;
    for (uint64_t u = j->lo; u < j->hi; u++) {
        const uint32_t b = (uint32_t)u;
        float x;
        memcpy(&x, &b, 4);
        const float a = expf(x), c = sf37_expf(x);
        const float s = host_sigmoid(x), t = sf37_sigmoid(x);
        uint32_t ua, uc, us, ut;
        memcpy(&ua, &a, 4); memcpy(&uc, &c, 4); memcpy(&us, &s, 4); memcpy(&ut, &t, 4);
        if (ua != uc && !(isnan(a) && isnan(c))) j->bad_exp++;
        if (us != ut && !(isnan(s) && isnan(t))) j->bad_sig++;
    }
    return nullptr;
}

int main() {
    const int nt = 8;
    pthread_t th[nt];
    job jb[nt];
    const uint64_t span = (1ull << 32) / nt;
    for (int i = 0; i < nt; i++) {
        jb[i] = {i * span, (i + 1) * span, 0, 0};
        pthread_create(&th[i], nullptr, run, &jb[i]);
    }
    uint64_t be = 0, bs = 0;
    for (int i = 0; i < nt; i++) {
        pthread_join(th[i], nullptr);
        be += jb[i].bad_exp;
        bs += jb[i].bad_sig;
    }
    printf("expf_mismatch %llu sigmoid_mismatch %llu\n", (unsigned long long)be, (unsigned long long)bs);
    return (be || bs) ? 1 : 0;
}
