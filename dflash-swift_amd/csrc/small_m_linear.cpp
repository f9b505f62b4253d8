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
 * device pointers owned by the caller; nothing is copied.  Errors are status codes.
 */
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

    static bool isEligible(const dfq_linear_desc& d) {
        return dfq_is_eligible(d.out_features, d.in_features, d.bits, d.group_size,
                               d.mode_affine, d.biases != nullptr) != 0;
    }
    static int tiles(int rows) { return dfq_tiles_for(rows); }
};

/* MLX's QuantizedLinear reduced to its arrays and call. */
class QuantizedLinear {
public:
    QuantizedLinear(dfq_ctx* ctx, const dfq_linear_desc& d) : ctx_(ctx), d_(d) {}
    virtual ~QuantizedLinear() = default;

    const dfq_linear_desc& desc() const { return d_; }
    dfq_ctx* ctx() const { return ctx_; }
    virtual bool isSmallM() const { return false; }

    /* The stock op's result dtype: MLX promotion of the input with the scales. */
    dfq_dtype outputDType(dfq_dtype x) const {
        return x == d_.dtype ? x : DFQ_F32;
    }

    virtual dfq_status callAsFunction(const void* x, dfq_dtype xdt, int rows, void* y,
                                      void* ws, size_t wsb, void* stream, int* took) {
        (void)ws;
        (void)wsb;
        if (took) *took = 0;
        if (!d_.biases)
            return dfq::fail(DFQ_ERR_UNSUPPORTED, "the generic path needs affine biases");
        return dfq_qmm_fallback(ctx_, x, d_.weight, d_.scales, d_.biases, d_.bias, y, rows,
                                d_.out_features, d_.in_features, d_.bits, d_.group_size, xdt,
                                d_.dtype, outputDType(xdt), stream);
    }

    virtual dfq_status workspaceBytes(int rows, size_t* bytes) const {
        (void)rows;
        *bytes = 0;
        return DFQ_OK;
    }

protected:
    dfq_ctx* ctx_;
    dfq_linear_desc d_;
};

/* SmallMQuantizedLinear: shares the wrapped layer's arrays (:243-252) and settles
 * eligibility once; callAsFunction takes the kernel only inside the window (:254-266). */
class SmallMQuantizedLinear final : public QuantizedLinear {
public:
    explicit SmallMQuantizedLinear(const QuantizedLinear& other)
        : QuantizedLinear(other.ctx(), other.desc()),
          kernelEligible_(SmallMQuantizedMatmul::isEligible(other.desc())) {
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
               xdt == DFQ_BF16 && d_.biases != nullptr && d_.dtype == DFQ_BF16;
    }

    dfq_status callAsFunction(const void* x, dfq_dtype xdt, int rows, void* y, void* ws,
                              size_t wsb, void* stream, int* took) override {
        if (!takesKernel(xdt, rows))
            return QuantizedLinear::callAsFunction(x, xdt, rows, y, ws, wsb, stream, took);
        if (took) *took = 1;
        return dfq_qmm(ctx_, x, d_.weight, d_.scales, d_.biases, d_.bias, y, rows,
                       d_.out_features, d_.in_features, d_.bits, d_.group_size, DFQ_BF16,
                       DFQ_BF16, DFQ_BF16, ws, wsb, stream);
    }

    dfq_status workspaceBytes(int rows, size_t* bytes) const override {
        *bytes = 0;
        if (!takesKernel(DFQ_BF16, rows)) return DFQ_OK;
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
        if (!dflash::SmallMQuantizedMatmul::isEligible(leaf->desc())) continue; // :310-311
        auto* swapped_leaf =                                                   // :313
            new dfq_linear{std::make_shared<dflash::SmallMQuantizedLinear>(*leaf)};
        model->owned.emplace_back(swapped_leaf);
        kv.second = swapped_leaf;
        ++swapped;
    }
    return swapped;                                                           // :315-316
}

}  // extern "C"
