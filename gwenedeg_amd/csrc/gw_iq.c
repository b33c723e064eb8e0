/* The i-quant codebooks on the device: expanded once per process from their compact form (gw_iq_tables.h) into the
 * byte layout the kernels read (gw_iq.h), then installed once per device. IQ1_S / IQ1_M's grid becomes two tables of
 * v = 8 grid + 1 and 8 grid - 1 (the integer form of grid +- 1/8, iquants.h:22-27), so its delta costs no arithmetic. */
#include <pthread.h>
#include <stdio.h>

#include "gw_internal.h"
#include "gw_iq_tables.h"

static uint64_t t_iq2xxs[256], t_iq2xs[512], t_iq2s[1024], t_iq1s[2][2048];
static uint32_t t_iq3xxs[256], t_iq3s[512];
static int expanded, dev_done[64];
static pthread_mutex_t mu = PTHREAD_MUTEX_INITIALIZER;

static void expand(void) {
    for (int i = 0; i < 256; i++) t_iq2xxs[i] = gw_iq2_entry(gw_iq2xxs_codes, i);
    for (int i = 0; i < 512; i++) t_iq2xs[i] = gw_iq2_entry(gw_iq2xs_codes, i);
    for (int i = 0; i < 1024; i++) t_iq2s[i] = gw_iq2_entry(gw_iq2s_codes, i);
    for (int i = 0; i < 256; i++) t_iq3xxs[i] = gw_iq3xxs_entry(i);
    for (int i = 0; i < 512; i++) t_iq3s[i] = gw_iq3s_entry(i);
    for (int i = 0; i < 2048; i++) {
        const uint64_t g = gw_iq1s_entry(i);
        uint64_t p = 0, n = 0;
        for (int j = 0; j < 8; j++) {
            const int v = 8 * (int)(int8_t)(g >> 8 * j);
            p |= (uint64_t)(uint8_t)(int8_t)(v + 1) << 8 * j;
            n |= (uint64_t)(uint8_t)(int8_t)(v - 1) << 8 * j;
        }
        t_iq1s[0][i] = p;
        t_iq1s[1][i] = n;
    }
    expanded = 1;
}

int gw_iq_init(char *err, size_t errlen) {
    int dev = 0, rc = RQ_OK;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return gw_hip_fail(err, errlen, "hipGetDevice", e);
    pthread_mutex_lock(&mu);
    if (!expanded) expand();
    if (dev >= 64) rc = RQ_ERR_STATE;
    else if (!dev_done[dev]) {
        int k = gw_g_set_iq(t_iq2xxs, t_iq2xs, t_iq2s, &t_iq1s[0][0], t_iq3xxs, t_iq3s);
        if (k) rc = gw_hip_fail(err, errlen, "hipMemcpyToSymbol (i-quant codebooks)", (hipError_t)k);
        else dev_done[dev] = 1;
    }
    pthread_mutex_unlock(&mu);
    if (rc == RQ_ERR_STATE && dev >= 64 && err && errlen) snprintf(err, errlen, "device %d: no i-quant codebooks", dev);
    return rc;
}
