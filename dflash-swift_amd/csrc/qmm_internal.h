/*
 * qmm_internal.h -- declarations shared by the runtime and the drop-in layer sources.
 */
#ifndef DFQ_QMM_INTERNAL_H
#define DFQ_QMM_INTERNAL_H

#include <cstddef>

#include "dflash_qmm.h"

namespace dfq {

/* The fast kernel's work split for one problem shape (see qmm_params.h). */
struct Plan {
    int kss = 0;        /* k per super-step                                  */
    int mt = 0;         /* row tiles of 8 (2 for 9..16 rows)                 */
    int T = 0;          /* column tiles of 16                                */
    int ch = 0;         /* super-steps per chunk (1, or 8 groups' worth)     */
    int chunks = 0;     /* chunks of K                                       */
    int SS = 0;         /* chunks in the largest k-block                     */
    int nkb = 0;        /* k-blocks (sizes differ by at most one chunk)      */
    int Gkb = 0;        /* workgroups per k-block                            */
    int nslot_kb = 0;   /* partial slots per tile per k-block                */
    int kr = 0;         /* k elements in the largest k-block                 */
    bool reduce = false; /* shared tiles summed by the second kernel         */
    bool aligned = false; /* workgroup ranges of whole tiles (two k-blocks)   */
    int rs = 0;         /* LDS bytes per staged x row                        */
    int xsum_off = 0;   /* LDS offset of the per-group x sums                */
    int part_off = 0;   /* LDS offset of the per-unit partial tiles          */
    int cnt_off = 0;    /* LDS offset of the tile arrival counters           */
    int gen_off = 0;    /* LDS offset of the partial slots' generations      */
    int tout_off = 0;   /* LDS offset of the finished tiles' fp32 sums        */
    int key_off = 0;    /* LDS offset of the per-row greedy-accept keys      */
    bool burst = false; /* tiles without a pair exchange leave at the end      */
    int ring = 0;       /* partial-tile slots (a ring over the take order)   */
    int umax = 0;       /* most units per workgroup                          */
    int lds_bytes = 0;  /* dynamic LDS requested per workgroup               */
    int lds_need = 0;   /* LDS bytes the layout uses                         */
    bool need_ws = false;
    size_t ws_bytes = 0;
};

dfq_status fail(dfq_status s, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
/* The device a context runs on. */
int ctx_device(const dfq_ctx* ctx);

/* Makes the context's device current for a scope and restores the previous one. */
class DeviceScope {
public:
    explicit DeviceScope(const dfq_ctx* ctx);
    ~DeviceScope();
    DeviceScope(const DeviceScope&) = delete;
    DeviceScope& operator=(const DeviceScope&) = delete;

private:
    int prev_ = -1;
    int dev_ = -1;
};
int kss_for(int bits, int gs);
/* Groups of a chunk of the c8 kernels (and of a unit of the packed layout). */
int chunk_groups(int bits, int gs);
bool make_plan(int M, int N, int K, int bits, int gs, int num_cus, size_t lds_max, Plan* pl);
/* The device address of the fixed scratch array (qmm_scratch.hip) on `device`, which must be
 * current; taken and cleared once per device. */
dfq_status scratch_setup(int device, void** out);
/* A layer whose only copy of the weight is `packed` (the packed layout, in memory the caller
 * keeps alive); d carries its shape, format, dtype and linear bias, and no MLX arrays. */
dfq_status make_packed_linear(dfq_ctx* ctx, const dfq_linear_desc& d, const void* packed,
                              dfq_linear** out);
dfq_status check_fast_args(const dfq_ctx* ctx, int M, int N, int K, int bits, int gs,
                           dfq_dtype xdt, dfq_dtype sdt, dfq_dtype ydt);

}  // namespace dfq

#endif
