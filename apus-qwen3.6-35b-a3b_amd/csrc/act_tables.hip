// act_tables.hip -- bf16-input activation tables.
//
// Every sigmoid on the hot path takes a bf16 value: the conv SiLU
// (c/gdn.h:19-33, of co = rnd(acc)), silu(z) of the gated RMSNorm
// (c/gdn.h:639-661), beta = rnd(sigmoid(b)) (c/gdn.h:366-370) and the
// attention output gate rnd(sigmoid(gate)) (c/attn.h:524-531). Each is
// therefore a function of a 16-bit code: the tables below hold it for all
// 65536 codes, computed once per device with the same correctly rounded
// arithmetic the kernels would otherwise evaluate per element (float64
// exp, one rounding), so a lookup gives bit-identical results for a
// fraction of the cost.
#include <hip/hip_runtime.h>

#include "apus_dev.h"
#include "apus_host.h"
#include "apus_rt.h"

using namespace apus;

namespace {

__global__ void k_fill_act_tables(uint16_t *__restrict__ silu_bf, float *__restrict__ silu_f,
                                  uint16_t *__restrict__ sig_bf) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= 65536) return;
    const float x = bf2f((uint16_t)c);
    const float sg = sigmoid_cr(x);
    silu_bf[c] = f2bf(x * sg);
    silu_f[c] = x * sg;
    sig_bf[c] = f2bf(sg);
}

ActTables g_tabs[16];
void *g_tab_mem[16];

}  // namespace

namespace apus {

const ActTables *act_tables() {
    const int dev = current_device();
    if (dev < 0 || dev >= 16) {
        set_error(kErrUnsupported, "device index %d out of range for the activation tables", dev);
        return nullptr;
    }
    if (g_tabs[dev].silu_bf) return &g_tabs[dev];
    void *p = nullptr;
    if (hipMalloc(&p, 65536 * (2 + 4 + 2)) != hipSuccess) {
        set_error(kErrHip, "hipMalloc of the activation tables failed");
        return nullptr;
    }
    ActTables t;
    t.silu_f = (float *)p;
    t.silu_bf = (uint16_t *)((char *)p + 65536 * 4);
    t.sig_bf = (uint16_t *)((char *)p + 65536 * 6);
    k_fill_act_tables<<<256, 256, 0, stream()>>>(const_cast<uint16_t *>(t.silu_bf),
                                                 const_cast<float *>(t.silu_f),
                                                 const_cast<uint16_t *>(t.sig_bf));
    if (launch_check("k_fill_act_tables") != kOk) {
        (void)hipFree(p);
        return nullptr;
    }
    g_tab_mem[dev] = p;
    g_tabs[dev] = t;
    return &g_tabs[dev];
}

}  // namespace apus
