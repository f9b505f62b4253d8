/*
 * small_m_linear.cpp -- the drop-in layer of the path, in C++ over the C ABI.
 *
 * Mirrors DFlashKit's Swift surface (paths relative to the reference repository root):
 *
 *   SmallMQuantizedMatmul            Sources/DFlashKit/SmallMQuantizedMatmul.swift:27-225
 *     .minimumRows ... .requiredGroupSize  (:32-47)
 *     .isEligible(_:)                (:193-201)
 *     .tiles(for:)                   (:205-207)
 *   SmallMQuantizedLinear            (:234-293)  a QuantizedLinear that shares the wrapped
 *                                                layer's arrays and routes verify-width,
 *                                                bf16 forwards through the fast kernel
 *   enableSmallMQuantizedMatmul(in:) (:303-317)  swaps every eligible leaf, idempotent,
 *                                                returns the count
 *
 * The module tree is reduced to what the swap needs: named leaf layers.  Layers hold
 * device pointers owned by the caller; nothing is copied, except by the opt-in
 * dfq_small_m_linear_pack.  Errors are status codes.
 *
 * A layer may also hold its weight in the packed layout (dfq_pack_weights): as a copy made by
 * dfq_small_m_linear_pack next to the MLX arrays, which the stock path keeps reading; or as
 * its only copy, loaded so by dfq_checkpoint_load_model_packed, when the stock path is the
 * fast kernel over that layout (16 rows a launch), there being no MLX arrays to hand to a
 * stock op.
 */
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "dflash_qmm.h"
#include "qmm_internal.h"

namespace dflash {

/* The static half of the reference type: the window constants and the gate. */
struct SmallMQuantizedMatmul {
    static constexpr int minimumRows = DFQ_MINIMUM_ROWS;
    static constexpr int maximumRows = DFQ_MAXIMUM_ROWS;
    static constexpr int rowsPerTile = DFQ_ROWS_PER_TILE;
    static constexpr int minimumOutputFeatures = DFQ_MINIMUM_OUTPUT_FEATURES;
    static constexpr int inputFeatureMultiple = DFQ_INPUT_FEATURE_MULTIPLE;
    static constexpr int requiredGroupSize = DFQ_REQUIRED_GROUP_SIZE;

    static bool isEligible(const dfq_linear_desc& d, bool hasBiases) {
        return dfq_is_eligible(d.out_features, d.in_features, d.bits, d.group_size,
                               d.mode_affine, hasBiases) != 0;
    }
    static int tiles(int rows) { return dfq_tiles_for(rows); }
};

/* A weight in the packed layout.  `owned` (a copy made by dfq_small_m_linear_pack) is freed
 * with the last layer that shares it; a loader's packed weight lives in its arena. */
struct PackedWeight {
    const void* ptr = nullptr;
    void* owned = nullptr;
    int device = -1;
    PackedWeight() = default;
    PackedWeight(const PackedWeight&) = delete;
    PackedWeight& operator=(const PackedWeight&) = delete;
    ~PackedWeight() {
        if (!owned) return;
        int prev = -1;
        if (hipGetDevice(&prev) == hipSuccess && prev != device) (void)hipSetDevice(device);
        (void)hipFree(owned);
        if (prev >= 0 && prev != device) (void)hipSetDevice(prev);
    }
};

/* MLX's QuantizedLinear reduced to its arrays and call. */
class QuantizedLinear {
public:
    QuantizedLinear(dfq_ctx* ctx, const dfq_linear_desc& d,
                    std::shared_ptr<PackedWeight> packed = nullptr)
        : ctx_(ctx), d_(d), packed_(std::move(packed)) {}
    virtual ~QuantizedLinear() = default;

    const dfq_linear_desc& desc() const { return d_; }
    dfq_ctx* ctx() const { return ctx_; }
    const std::shared_ptr<PackedWeight>& packed() const { return packed_; }
    void setPacked(std::shared_ptr<PackedWeight> pw) { packed_ = std::move(pw); }
    /* Only the packed copy: no MLX arrays (dfq_checkpoint_load_model_packed). */
    bool packedOnly() const { return packed_ && !d_.weight; }
    bool hasBiases() const { return d_.biases != nullptr || packedOnly(); }
    bool eligible() const { return SmallMQuantizedMatmul::isEligible(d_, hasBiases()); }
    virtual bool isSmallM() const { return false; }

    /* The stock op's result dtype: MLX promotion of the input with the scales. */
    dfq_dtype outputDType(dfq_dtype x) const {
        return x == d_.dtype ? x : DFQ_F32;
    }

    virtual dfq_status callAsFunction(const void* x, dfq_dtype xdt, int rows, void* y,
                                      void* ws, size_t wsb, void* stream, int* took) {
        if (took) *took = 0;
        if (packedOnly()) return packedSlices(x, xdt, rows, y, ws, wsb, stream);
        if (!d_.biases)
            return dfq::fail(DFQ_ERR_UNSUPPORTED, "the generic path needs affine biases");
        return dfq_qmm_fallback(ctx_, x, d_.weight, d_.scales, d_.biases, d_.bias, y, rows,
                                d_.out_features, d_.in_features, d_.bits, d_.group_size, xdt,
                                d_.dtype, outputDType(xdt), stream);
    }

    virtual dfq_status workspaceBytes(int rows, size_t* bytes) const {
        *bytes = 0;
        if (!packedOnly()) return DFQ_OK;
        /* the stock path of a packed-only layer: launches of up to 16 rows */
        for (int r : {std::min(rows, kSlice), rows % kSlice}) {
            size_t b = 0;
            if (r < 1) continue;
            dfq_status s = dfq_qmm_workspace_bytes(ctx_, r, d_.out_features, d_.in_features,
                                                   d_.bits, d_.group_size, &b);
            if (s) return s;
            *bytes = std::max(*bytes, b);
        }
        return DFQ_OK;
    }

protected:
    static constexpr int kSlice = DFQ_MAXIMUM_ROWS;

    /* The fast kernel over the packed copy, up to 16 rows a launch: the stock path of a layer
     * that has no MLX arrays (x, scales and y in the one dtype the pack holds). */
    dfq_status packedSlices(const void* x, dfq_dtype xdt, int rows, void* y, void* ws,
                            size_t wsb, void* stream) const {
        if (xdt != d_.dtype)
            return dfq::fail(DFQ_ERR_UNSUPPORTED,
                             "a packed layer takes x in the dtype of its scales (%d), not %d",
                             (int)d_.dtype, (int)xdt);
        const size_t xrow = (size_t)d_.in_features * 2, yrow = (size_t)d_.out_features * 2;
        for (int r0 = 0; r0 < rows; r0 += kSlice) {
            const int r = std::min(kSlice, rows - r0);
            dfq_status s = dfq_qmm_packed(ctx_, (const char*)x + r0 * xrow, packed_->ptr, d_.bias,
                                          (char*)y + r0 * yrow, r, d_.out_features,
                                          d_.in_features, d_.bits, d_.group_size, d_.dtype, ws,
                                          wsb, stream);
            if (s) return s;
        }
        return DFQ_OK;
    }

    dfq_ctx* ctx_;
    dfq_linear_desc d_;
    std::shared_ptr<PackedWeight> packed_;
};

/* SmallMQuantizedLinear: shares the wrapped layer's arrays (:243-252) and settles
 * eligibility once; callAsFunction takes the kernel only inside the window (:254-266). */
class SmallMQuantizedLinear final : public QuantizedLinear {
public:
    explicit SmallMQuantizedLinear(const QuantizedLinear& other)
        : QuantizedLinear(other.ctx(), other.desc(), other.packed()),
          kernelEligible_(other.eligible()) {
        /* The reference gate says nothing of the kernel's own limits (weights under 2 GiB,
         * a work split for the shape).  Rows the fast kernel cannot take fall through to the
         * stock op like any other ineligible call (:254-266), decided once here. */
        if (kernelEligible_ && ctx_)
            for (int r = SmallMQuantizedMatmul::minimumRows; r <= SmallMQuantizedMatmul::maximumRows; ++r)
                if (dfq_qmm_supported(ctx_, r, d_.out_features, d_.in_features, d_.bits,
                                      d_.group_size, DFQ_BF16, DFQ_BF16, DFQ_BF16))
                    rowsFit_ |= 1u << r;
    }

    bool isSmallM() const override { return true; }

    bool takesKernel(dfq_dtype xdt, int rows) const {
        return kernelEligible_ && rows >= SmallMQuantizedMatmul::minimumRows &&
               rows <= SmallMQuantizedMatmul::maximumRows && ((rowsFit_ >> rows) & 1u) &&
               xdt == DFQ_BF16 && hasBiases() && d_.dtype == DFQ_BF16;
    }

    dfq_status callAsFunction(const void* x, dfq_dtype xdt, int rows, void* y, void* ws,
                              size_t wsb, void* stream, int* took) override {
        if (!takesKernel(xdt, rows))
            return QuantizedLinear::callAsFunction(x, xdt, rows, y, ws, wsb, stream, took);
        if (took) *took = 1;
        if (packed_)
            return dfq_qmm_packed(ctx_, x, packed_->ptr, d_.bias, y, rows, d_.out_features,
                                  d_.in_features, d_.bits, d_.group_size, DFQ_BF16, ws, wsb,
                                  stream);
        return dfq_qmm(ctx_, x, d_.weight, d_.scales, d_.biases, d_.bias, y, rows,
                       d_.out_features, d_.in_features, d_.bits, d_.group_size, DFQ_BF16,
                       DFQ_BF16, DFQ_BF16, ws, wsb, stream);
    }

    dfq_status workspaceBytes(int rows, size_t* bytes) const override {
        *bytes = 0;
        if (!takesKernel(DFQ_BF16, rows)) return QuantizedLinear::workspaceBytes(rows, bytes);
        return dfq_qmm_workspace_bytes(ctx_, rows, d_.out_features, d_.in_features, d_.bits,
                                       d_.group_size, bytes);
    }

private:
    bool kernelEligible_;
    uint32_t rowsFit_ = 0;  /* bit r: the fast kernel has a split for r rows of this layer */
};

}  // namespace dflash

/* ---- C handles ------------------------------------------------------------------------ */

struct dfq_linear {
    std::shared_ptr<dflash::QuantizedLinear> impl;
};

/* The model owns one handle per leaf it has ever held: dfq_model_leaf hands out borrowed
 * handles, which stay valid (describing the layer they named) until the model is destroyed,
 * also after a swap or set_leaf replaced that leaf. */
struct dfq_model {
    std::map<std::string, dfq_linear*> leaves;
    std::vector<std::unique_ptr<dfq_linear>> owned;
};

dfq_status dfq::make_packed_linear(dfq_ctx* ctx, const dfq_linear_desc& d, const void* packed,
                                   dfq_linear** out) {
    if (!packed || !out || d.weight || d.scales || d.biases)
        return dfq::fail(DFQ_ERR_INVALID_ARGUMENT, "a packed layer has no MLX arrays");
    auto pw = std::make_shared<dflash::PackedWeight>();
    pw->ptr = packed;
    *out = new dfq_linear{std::make_shared<dflash::QuantizedLinear>(ctx, d, std::move(pw))};
    return DFQ_OK;
}

extern "C" {

dfq_status dfq_linear_describe(const dfq_linear* lin, dfq_linear_desc* out) {
    if (!lin || !out) return dfq::fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    *out = lin->impl->desc();
    return DFQ_OK;
}

dfq_status dfq_linear_create(dfq_ctx* ctx, const dfq_linear_desc* desc, dfq_linear** out) {
    /* ctx may be NULL: such a layer can be inspected and swapped but not called. */
    if (!desc || !out) return dfq::fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    const dfq_linear_desc& d = *desc;
    if (!d.weight || !d.scales)
        return dfq::fail(DFQ_ERR_INVALID_ARGUMENT, "weight and scales are required");
    if (d.out_features < 1 || d.in_features < 1 || d.bits < 1 || d.group_size < 1)
        return dfq::fail(DFQ_ERR_INVALID_ARGUMENT, "shape and format must be positive");
    if (d.in_features % d.group_size)
        return dfq::fail(DFQ_ERR_INVALID_ARGUMENT, "group size %d does not divide in=%d",
                         d.group_size, d.in_features);
    if (d.dtype != DFQ_BF16 && d.dtype != DFQ_F16 && d.dtype != DFQ_F32)
        return dfq::fail(DFQ_ERR_INVALID_ARGUMENT, "bad dtype");
    *out = new dfq_linear{std::make_shared<dflash::QuantizedLinear>(ctx, d)};
    return DFQ_OK;
}

dfq_status dfq_small_m_linear_create(dfq_linear* other, dfq_linear** out) {
    if (!other || !out) return dfq::fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    *out = new dfq_linear{std::make_shared<dflash::SmallMQuantizedLinear>(*other->impl)};
    return DFQ_OK;
}

dfq_status dfq_linear_destroy(dfq_linear* lin) {
    delete lin;
    return DFQ_OK;
}

int dfq_linear_is_small_m(const dfq_linear* lin) { return lin && lin->impl->isSmallM(); }

const void* dfq_linear_packed(const dfq_linear* lin) {
    return lin && lin->impl->packed() ? lin->impl->packed()->ptr : nullptr;
}

dfq_status dfq_small_m_linear_pack(dfq_linear* lin, void* stream) {
    if (!lin) return dfq::fail(DFQ_ERR_INVALID_ARGUMENT, "null layer");
    auto& L = *lin->impl;
    if (!L.isSmallM())
        return dfq::fail(DFQ_ERR_INVALID_ARGUMENT,
                         "only a SmallMQuantizedLinear takes a packed copy");
    if (L.packed()) return DFQ_OK;
    if (!L.ctx()) return dfq::fail(DFQ_ERR_STATE, "layer was created without a context");
    const dfq_linear_desc& d = L.desc();
    if (!L.eligible() || !d.biases || d.dtype != DFQ_BF16)
        return dfq::fail(DFQ_ERR_UNSUPPORTED,
                         "a packed copy serves the fast kernel's bf16 calls of an eligible layer");
    size_t bytes = 0;
    dfq_status s = dfq_packed_bytes(d.out_features, d.in_features, d.bits, d.group_size, &bytes);
    if (s) return s;
    auto pw = std::make_shared<dflash::PackedWeight>();
    pw->device = dfq::ctx_device(L.ctx());
    dfq::DeviceScope g(L.ctx());
    hipError_t e = hipMalloc(&pw->owned, bytes);
    if (e != hipSuccess)
        return dfq::fail(DFQ_ERR_HIP, "packed copy of %zu bytes: %s", bytes, hipGetErrorString(e));
    pw->ptr = pw->owned;
    s = dfq_pack_weights(L.ctx(), d.weight, d.scales, d.biases, d.out_features, d.in_features,
                         d.bits, d.group_size, pw->owned, stream);
    if (s) return s;
    if ((e = hipStreamSynchronize((hipStream_t)stream)) != hipSuccess)
        return dfq::fail(DFQ_ERR_HIP, "packing: %s", hipGetErrorString(e));
    L.setPacked(std::move(pw));
    return DFQ_OK;
}

dfq_dtype dfq_linear_output_dtype(const dfq_linear* lin, dfq_dtype x_dtype) {
    /* Both paths return MLX's promotion of (x, scales): the kernel path only runs when
     * both are bf16, where the promotion is bf16 as well. */
    return lin ? lin->impl->outputDType(x_dtype) : x_dtype;
}

dfq_status dfq_linear_forward(dfq_linear* lin, const void* x, dfq_dtype x_dtype, int rows,
                              void* y, void* ws, size_t wsb, void* stream, int* took_kernel) {
    if (!lin) return dfq::fail(DFQ_ERR_INVALID_ARGUMENT, "null layer");
    if (!lin->impl->ctx()) return dfq::fail(DFQ_ERR_STATE, "layer was created without a context");
    if (rows < 1) return dfq::fail(DFQ_ERR_INVALID_ARGUMENT, "rows must be >= 1");
    return lin->impl->callAsFunction(x, x_dtype, rows, y, ws, wsb, stream, took_kernel);
}

dfq_status dfq_linear_workspace_bytes(dfq_linear* lin, int rows, size_t* bytes) {
    if (!lin || !bytes) return dfq::fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    if (!lin->impl->ctx()) return dfq::fail(DFQ_ERR_STATE, "layer was created without a context");
    return lin->impl->workspaceBytes(rows, bytes);
}

dfq_status dfq_model_create(dfq_model** out) {
    if (!out) return dfq::fail(DFQ_ERR_INVALID_ARGUMENT, "null out");
    *out = new dfq_model();
    return DFQ_OK;
}

dfq_status dfq_model_destroy(dfq_model* model) {
    delete model;
    return DFQ_OK;
}

dfq_status dfq_model_set_leaf(dfq_model* model, const char* path, dfq_linear* lin) {
    if (!model || !path || !lin) return dfq::fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    /* A handle the model already owns (set at another path, as a tied layer is, or one that
     * dfq_model_leaf returned) is only pointed at again: owning it twice would free it twice
     * when the model is destroyed. */
    bool owned = false;
    for (const auto& o : model->owned)
        if (o.get() == lin) owned = true;
    if (!owned) model->owned.emplace_back(lin);
    model->leaves[path] = lin;
    return DFQ_OK;
}

dfq_linear* dfq_model_leaf(dfq_model* model, const char* path) {
    if (!model || !path) return nullptr;
    auto it = model->leaves.find(path);
    return it == model->leaves.end() ? nullptr : it->second;
}

int dfq_model_leaf_count(const dfq_model* model) {
    return model ? (int)model->leaves.size() : 0;
}

int dfq_enable_small_m_quantized_matmul(dfq_model* model) {
    if (!model) {
        dfq::fail(DFQ_ERR_INVALID_ARGUMENT, "null model");
        return -1;
    }
    int swapped = 0;
    for (auto& kv : model->leaves) {
        const auto& leaf = kv.second->impl;
        if (leaf->isSmallM()) continue;                                       // :309
        if (!leaf->eligible()) continue;                                      // :310-311
        auto* swapped_leaf =                                                   // :313
            new dfq_linear{std::make_shared<dflash::SmallMQuantizedLinear>(*leaf)};
        model->owned.emplace_back(swapped_leaf);
        kv.second = swapped_leaf;
        ++swapped;
    }
    return swapped;                                                           // :315-316
}

}  // extern "C"
