// Dispatch validation: the checks of CpuDevice::dispatch
// (crates/backends/backend-cpu/src/device.rs) restated for the HIP device,
// with the same order and the same static error strings, plus the checks the
// reference kernels make before their first write (reference/*.rs). The
// quantized-operand rules have no reference counterpart (see
// sl_hip_bind_quantized in starlight_hip.h).
#include <cstring>

#include "plan.h"

namespace slhip {
namespace {

// Operator signature summary (sl-ir OpCode::signature, ARCH-0004 §5.2):
// number of input ports (scalar ports included), how many of them are
// scalars, and the number of outputs. Scalar port positions follow
// executor.rs:1008-1009, 1172, 1195, 1298.
struct SignatureInfo {
    uint8_t inputs;
    uint8_t scalar_ports;
    uint8_t outputs;
};

constexpr SignatureInfo kSignatures[kOpCount] = {
    {2, 0, 1},  // MatMulNT
    {2, 0, 1},  // MatMulNN
    {1, 0, 1},  // Softmax
    {3, 2, 1},  // SoftmaxCausal: X, seq_len, past_len
    {2, 0, 1},  // RmsNorm
    {2, 0, 1},  // Rope: X, positions
    {1, 0, 1},  // Silu
    {2, 0, 1},  // Mul
    {2, 0, 1},  // Add
    {1, 0, 1},  // Scale
    {2, 0, 1},  // Gather: table, ids
    {2, 1, 1},  // LastToken: X, seq_len
    {3, 1, 0},  // KvAppend: K, V, past_len (no output)
    {1, 0, 1},  // SplitHeads
    {1, 0, 1},  // MergeHeads
    {4, 1, 1},  // CausalAttention: Q, K, V, past_len
    {4, 0, 1},  // SwiGlu: X, gate, up, down
    {3, 0, 1},  // RmsNormMatMul: X, weight, matrix
};

// Dims (device.rs:708-770): rank plus concrete extents.
struct Dims {
    size_t rank = 0;
    uint64_t e[kMaxRank] = {};

    bool dim(size_t i, uint64_t* out, Error* err) const {
        if (i < rank) {
            *out = e[i];
            return true;
        }
        *err = Error::execution("operator rank is too small");
        return false;
    }
    bool last(uint64_t* out, Error* err) const {
        if (rank == 0) {
            *err = Error::execution("operator requires at least one dimension");
            return false;
        }
        *out = e[rank - 1];
        return true;
    }
    bool product(size_t end, uint64_t* out, Error* err) const {
        if (end > rank) {
            *err = Error::execution("operator rank is too small");
            return false;
        }
        uint64_t p = 1;
        for (size_t i = 0; i < end; ++i) {
            if (e[i] != 0 && p > UINT64_MAX / e[i]) {
                *err = Error::overflow();
                return false;
            }
            p *= e[i];
        }
        *out = p;
        return true;
    }
    bool same_as(const Dims& o) const {
        if (rank != o.rank) return false;
        for (size_t i = 0; i < rank; ++i)
            if (e[i] != o.e[i]) return false;
        return true;
    }
};

bool dims_of(const sl_value& v, Dims* d, Error* err) {
    if (v.rank > kMaxRank) {
        *err = Error::overflow();
        return false;
    }
    d->rank = v.rank;
    for (size_t i = 0; i < v.rank; ++i) d->e[i] = v.dims[i];
    return true;
}

bool checked_mul(uint64_t a, uint64_t b, uint64_t* out, Error* err) {
    if (a != 0 && b > UINT64_MAX / a) {
        *err = Error::overflow();
        return false;
    }
    *out = a * b;
    return true;
}

#define TRY(expr)              \
    do {                       \
        if (!(expr)) return false; \
    } while (0)

#define FAIL(why)                        \
    do {                                 \
        *err = Error::execution(why);    \
        return false;                    \
    } while (0)

// validate_alignment-free part of validate_call (device.rs:224-286).
bool validate_call(const sl_op& op, const sl_value* input_values, size_t n_inputs, size_t n_outputs,
                   size_t n_scalars, Error* err) {
    if (n_inputs > kMaxInputs || n_outputs > kMaxOutputs) FAIL("too many command ports");
    const SignatureInfo& sig = kSignatures[op.code];
    size_t state_ports = 0;
    for (size_t i = 0; i < n_inputs; ++i)
        if (input_values[i].role == SL_ROLE_STATE) ++state_ports;
    bool stateful = op.code == SL_OP_KV_APPEND || op.code == SL_OP_CAUSAL_ATTENTION;
    if (stateful) {
        if (state_ports != 1) FAIL("stateful operator requires exactly one State input");
    } else if (state_ports != 0) {
        FAIL("stateless operator received a State input");
    }
    size_t expected_inputs = sig.inputs - sig.scalar_ports + state_ports;
    if (n_inputs != expected_inputs) FAIL("input buffer count does not match the operator signature");
    if (n_outputs != sig.outputs) FAIL("output count does not match the operator signature");
    if (n_scalars != sig.scalar_ports) FAIL("scalar count does not match the operator signature");
    return true;
}

// check_range (device.rs:326-339).
bool check_range(const sl_buffer_ref& r, uint64_t capacity, Error* err) {
    if (r.offset > UINT64_MAX - r.len) {
        *err = Error::overflow();
        return false;
    }
    if (r.offset + r.len > capacity) {
        *err = Error::invalid_range(r.buffer, r.offset, r.len);
        return false;
    }
    return true;
}

// validate_port (device.rs:288-324), extended with the group-quantized
// operand rules.
bool validate_port(const BufferView& buffers, const sl_buffer_ref& r, const sl_value& v, bool output,
                   QuantOperand* quant, Error* err) {
    if (v.role == SL_ROLE_SCALAR) FAIL("scalar operands must be passed through the scalars argument");
    Dims d;
    TRY(dims_of(v, &d, err));
    uint64_t elements;
    TRY(d.product(d.rank, &elements, err));
    const sl_buffer_desc* desc = buffers.get(r.buffer);

    if (v.encoding == SL_ENCODING_OPAQUE_QUANTIZED) {
        *err = Error::unimplemented("opaque quantized encodings cannot be executed");
        return false;
    }
    if (v.encoding == SL_ENCODING_GROUPWISE_QUANTIZED) {
        if (output) FAIL("quantized values cannot be command outputs");
        if (v.role != SL_ROLE_PARAM) FAIL("only Param values may use a quantized encoding");
        if (v.dtype != SL_DTYPE_F32) {
            *err = Error::unimplemented("dtype is not supported by HipDevice");
            return false;
        }
        if (v.qformat != SL_QFORMAT_INT4 && v.qformat != SL_QFORMAT_INT8) {
            *err = Error::unimplemented("quantization format is not supported by HipDevice");
            return false;
        }
        if (d.rank != 2) FAIL("quantized weights must have shape [n, k]");
        if (desc == nullptr || desc->kind != SL_BUFFER_U32) {
            *err = Error::invalid_buffer(r.buffer);
            return false;
        }
        if (!desc->quantized) FAIL("quantized operand buffer has no bound scales");
        if (desc->qformat != v.qformat || desc->group_size != v.group_size || desc->qn != d.e[0] ||
            desc->qk != d.e[1])
            FAIL("quantized operand does not match its buffer binding");
        if (quant_payload_words(v.qformat, d.e[0], d.e[1]) != r.len)
            FAIL("BufferRef length does not match the quantized payload size");
        TRY(check_range(r, desc->elements, err));
        quant->present = true;
        quant->format = v.qformat;
        quant->group = v.group_size;
        quant->n = d.e[0];
        quant->k = d.e[1];
        return true;
    }

    if (elements != r.len) FAIL("BufferRef length does not match the value element count");
    switch (v.dtype) {
        case SL_DTYPE_F32:
            if (desc == nullptr || desc->kind != SL_BUFFER_F32) {
                *err = Error::invalid_buffer(r.buffer);
                return false;
            }
            return check_range(r, desc->elements, err);
        case SL_DTYPE_U32:
            if (output) FAIL("integer command outputs are not supported");
            if (desc == nullptr || desc->kind != SL_BUFFER_U32) {
                *err = Error::invalid_buffer(r.buffer);
                return false;
            }
            return check_range(r, desc->elements, err);
        default:
            *err = Error::unimplemented("dtype is not supported by HipDevice");
            return false;
    }
}

// ranges_overlap (device.rs:370-377).
bool ranges_overlap(const sl_buffer_ref& a, const sl_buffer_ref& b) {
    if (a.buffer != b.buffer) return false;
    uint64_t a_end = a.offset > UINT64_MAX - a.len ? UINT64_MAX : a.offset + a.len;
    uint64_t b_end = b.offset > UINT64_MAX - b.len ? UINT64_MAX : b.offset + b.len;
    return a.offset < b_end && b.offset < a_end;
}

// check_disjoint (device.rs:341-368).
bool check_disjoint(const sl_buffer_ref* in, size_t n_in, const sl_buffer_ref* out, size_t n_out,
                    Error* err) {
    for (size_t i = 0; i < n_in; ++i) {
        for (size_t j = i + 1; j < n_in; ++j)
            if (ranges_overlap(in[i], in[j])) FAIL("one command aliases overlapping input ranges");
        for (size_t j = 0; j < n_out; ++j)
            if (ranges_overlap(in[i], out[j]))
                FAIL("a command output aliases an overlapping input range");
    }
    for (size_t i = 0; i < n_out; ++i)
        for (size_t j = i + 1; j < n_out; ++j)
            if (ranges_overlap(out[i], out[j])) FAIL("one command aliases overlapping output ranges");
    return true;
}

// broadcast_batch (device.rs:1334-1355).
bool broadcast_batch(uint64_t left, uint64_t right, uint64_t* out, Error* err) {
    if (left == right) {
        *out = left;
        return true;
    }
    if (left == 0 || right == 0) {
        if ((left > right ? left : right) <= 1) {
            *out = 0;
            return true;
        }
        FAIL("matmul batch dimensions are not broadcastable");
    }
    if (left == 1) {
        *out = right;
        return true;
    }
    if (right == 1) {
        *out = left;
        return true;
    }
    FAIL("matmul batch dimensions are not broadcastable");
}

// matmul_geometry (device.rs:1301-1332).
bool matmul_geometry(const Dims& l, const Dims& r, const Dims& o, bool transposed, Plan* p, Error* err) {
    if (l.rank < 2 || r.rank < 2 || o.rank < 2) FAIL("matmul operands and output must have rank at least 2");
    uint64_t m, k, rk, n;
    TRY(l.dim(l.rank - 2, &m, err));
    TRY(l.dim(l.rank - 1, &k, err));
    if (transposed) {
        TRY(r.dim(r.rank - 1, &rk, err));
        TRY(r.dim(r.rank - 2, &n, err));
    } else {
        TRY(r.dim(r.rank - 2, &rk, err));
        TRY(r.dim(r.rank - 1, &n, err));
    }
    if (k != rk) FAIL("matmul reduction dimensions must match");
    uint64_t ba, bb, batch;
    TRY(l.product(l.rank - 2, &ba, err));
    TRY(r.product(r.rank - 2, &bb, err));
    TRY(broadcast_batch(ba, bb, &batch, err));
    uint64_t om, on, ob;
    TRY(o.dim(o.rank - 2, &om, err));
    TRY(o.dim(o.rank - 1, &on, err));
    if (om != m || on != n) FAIL("matmul output shape must be m x n");
    TRY(o.product(o.rank - 2, &ob, err));
    if (ob != batch) FAIL("matmul output batch must match the operands");
    p->batch_a = ba;
    p->batch_b = bb;
    p->batch = batch;
    p->m = m;
    p->k = k;
    p->n = n;
    return true;
}

// row_geometry (device.rs:1409-1413).
bool row_geometry(const Dims& in, uint64_t* rows, uint64_t* hidden, Error* err) {
    TRY(in.last(hidden, err));
    return in.product(in.rank - 1, rows, err);
}

// check_state_geometry (device.rs:1466-1488).
bool check_state_geometry(const Dims& s, uint64_t batch, uint64_t kv_heads, uint64_t head_dim,
                          uint64_t layer, Plan* p, Error* err) {
    if (s.rank != 6 || s.e[0] != batch || s.e[2] != 2 || s.e[4] != kv_heads || s.e[5] != head_dim)
        FAIL("KV cache shape must be [batch, layers, 2, max_seq, kv_heads, head_dim]");
    if (layer >= s.e[1]) FAIL("attention layer is out of range");
    p->layers = s.e[1];
    p->max_seq = s.e[3];
    return true;
}

bool scalar_at(const uint32_t* scalars, size_t n, size_t i, uint64_t* out, Error* err) {
    if (i >= n) FAIL("operator is missing a scalar input");
    *out = scalars[i];
    return true;
}

// Rejects quantized operands on ports that cannot take them.
bool only_quantized_at(const QuantOperand* q, size_t n_inputs, uint32_t allowed_mask, Error* err) {
    for (size_t i = 0; i < n_inputs; ++i)
        if (q[i].present && !(allowed_mask & (1u << i))) {
            *err = Error::unimplemented("quantized operand is not supported on this port");
            return false;
        }
    return true;
}

// A quantized [n, k] weight must agree with the geometry using it.
bool quant_matches(const QuantOperand& q, uint64_t n, uint64_t k, Error* err) {
    if (!q.present) return true;
    if (q.group == 0 || q.k % q.group != 0) FAIL("quantized k must be a positive multiple of group_size");
    if (q.n != n || q.k != k) FAIL("quantized weight shape does not match the operator geometry");
    return true;
}

// The per-op part of run_op (device.rs:773-1227) plus the InvalidShape checks
// of the reference kernels it calls.
bool op_geometry(const sl_op& op, const sl_value* iv, size_t n_in, const sl_value* ov, size_t n_out,
                 const uint32_t* scalars, size_t n_scalars, Plan* p, Error* err) {
    Dims in0, in1, in2, in3, out;
    auto input = [&](size_t i, Dims* d) -> bool {
        if (i >= n_in) FAIL("operator is missing an input value");
        return dims_of(iv[i], d, err);
    };
    auto output = [&](Dims* d) -> bool {
        if (n_out == 0) FAIL("operator is missing an output value");
        return dims_of(ov[0], d, err);
    };
    switch (op.code) {
        case SL_OP_MATMUL_NT:
        case SL_OP_MATMUL_NN: {
            TRY(only_quantized_at(p->quant, n_in, op.code == SL_OP_MATMUL_NT ? 0x2u : 0u, err));
            TRY(input(0, &in0));
            TRY(input(1, &in1));
            TRY(output(&out));
            TRY(matmul_geometry(in0, in1, out, op.code == SL_OP_MATMUL_NT, p, err));
            return quant_matches(p->quant[1], p->n, p->k, err);
        }
        case SL_OP_SOFTMAX:
        case SL_OP_SOFTMAX_CAUSAL: {
            bool causal = op.code == SL_OP_SOFTMAX_CAUSAL;
            TRY(input(0, &in0));
            TRY(output(&out));
            if (!in0.same_as(out))
                FAIL(causal ? "softmax_causal output shape must match its input"
                            : "softmax output shape must match its input");
            TRY(in0.last(&p->cols, err));
            TRY(in0.product(in0.rank - 1, &p->rows, err));
            if (!causal) {
                // reference/softmax.rs:20-24
                if (p->rows == 0 || p->cols == 0) FAIL("softmax requires nonzero rows and cols");
                return true;
            }
            TRY(scalar_at(scalars, n_scalars, 0, &p->seq, err));
            TRY(scalar_at(scalars, n_scalars, 1, &p->past_len, err));
            // reference/softmax.rs:68-91
            if (p->rows == 0 || p->cols == 0) FAIL("softmax_causal requires nonzero rows and cols");
            if (p->seq == 0) FAIL("softmax_causal requires a nonzero seq");
            if (p->cols != p->past_len + p->seq) FAIL("softmax_causal requires cols == past_len + seq");
            if (p->rows % p->seq != 0) FAIL("softmax_causal requires rows to be a multiple of seq");
            return true;
        }
        case SL_OP_RMS_NORM: {
            TRY(input(0, &in0));
            TRY(input(1, &in1));
            TRY(output(&out));
            TRY(row_geometry(in0, &p->rows, &p->hidden, err));
            if (in1.rank != 1 || in1.e[0] != p->hidden) FAIL("rms_norm weight shape must be [hidden]");
            if (!in0.same_as(out)) FAIL("rms_norm output shape must match its input");
            if (p->hidden == 0) FAIL("rms_norm requires a nonzero hidden size");  // norm.rs:35-39
            p->eps = op.eps;
            return true;
        }
        case SL_OP_ROPE: {
            TRY(input(0, &in0));
            TRY(input(1, &in1));
            TRY(output(&out));
            // rope_geometry (device.rs:1415-1428)
            if (in0.rank == 4) {
                p->batch = in0.e[0];
                p->heads = in0.e[1];
                p->seq = in0.e[2];
                p->head_dim = in0.e[3];
            } else if (in0.rank == 3) {
                p->batch = in0.e[0];
                p->heads = 1;
                p->seq = in0.e[1];
                p->head_dim = in0.e[2];
            } else {
                FAIL("rope input must have rank 3 or 4");
            }
            if (in1.rank != 2 || in1.e[0] != p->batch || in1.e[1] != p->seq)
                FAIL("rope positions shape must be [batch, seq]");
            if (!in0.same_as(out)) FAIL("rope output shape must match its input");
            if (p->head_dim == 0 || p->head_dim % 2 != 0)  // rope.rs:16-20
                FAIL("head_dim must be a positive even number");
            p->theta = op.theta;
            p->rope_variant = op.rope_variant;
            if (op.rope_variant > SL_ROPE_GPTJ) {
                *err = Error::unimplemented("rope variant is not supported by HipDevice");
                return false;
            }
            return true;
        }
        case SL_OP_SILU:
        case SL_OP_SCALE: {
            TRY(input(0, &in0));
            TRY(output(&out));
            if (!in0.same_as(out))
                FAIL(op.code == SL_OP_SILU ? "silu output shape must match its input"
                                           : "scale output shape must match its input");
            TRY(in0.product(in0.rank, &p->len, err));
            p->factor = op.factor;
            return true;
        }
        case SL_OP_MUL:
        case SL_OP_ADD: {
            TRY(input(0, &in0));
            TRY(input(1, &in1));
            TRY(output(&out));
            if (!in0.same_as(in1) || !in0.same_as(out))
                FAIL("mul/add operands and output must have identical shapes");
            return in0.product(in0.rank, &p->len, err);
        }
        case SL_OP_GATHER: {
            TRY(input(0, &in0));
            TRY(input(1, &in1));
            TRY(output(&out));
            if (in0.rank != 2) FAIL("gather table must have shape [vocab, hidden]");
            p->vocab = in0.e[0];
            p->hidden = in0.e[1];
            TRY(in1.product(in1.rank, &p->rows, err));
            if (out.rank != in1.rank + 1) FAIL("gather output rank must be the id rank plus one");
            for (size_t i = 0; i < in1.rank; ++i)
                if (out.e[i] != in1.e[i]) FAIL("gather output prefix must match the id shape");
            uint64_t width;
            TRY(out.last(&width, err));
            if (width != p->hidden) FAIL("gather output width must equal hidden");
            return true;
        }
        case SL_OP_LAST_TOKEN: {
            TRY(input(0, &in0));
            TRY(output(&out));
            TRY(scalar_at(scalars, n_scalars, 0, &p->seq_len, err));
            if (in0.rank != 3 || out.rank != 2) FAIL("last_token shapes must be [B, M, H] -> [B, H]");
            p->batch = in0.e[0];
            p->seq = in0.e[1];
            p->hidden = in0.e[2];
            if (out.e[0] != p->batch || out.e[1] != p->hidden)
                FAIL("last_token output shape must be [batch, hidden]");
            if (p->seq_len < 1 || p->seq_len > p->seq)  // layout.rs:78-82
                FAIL("last_token requires 1 <= seq_len <= seq");
            return true;
        }
        case SL_OP_KV_APPEND: {
            TRY(input(0, &in0));
            TRY(input(1, &in1));
            TRY(scalar_at(scalars, n_scalars, 0, &p->past_len, err));
            p->layer = op.layer;
            // attention_kv_geometry (device.rs:1453-1464)
            if (in0.rank != 4 || in1.rank != 4) FAIL("kv_append key/value must have rank 4");
            if (!in0.same_as(in1)) FAIL("kv_append key and value shapes must match");
            p->batch = in0.e[0];
            p->kv_heads = in0.e[1];
            p->seq = in0.e[2];
            p->head_dim = in0.e[3];
            if (p->state_index < 0) FAIL("kv_append requires a State input");
            Dims st;
            TRY(dims_of(iv[p->state_index], &st, err));
            TRY(check_state_geometry(st, p->batch, p->kv_heads, p->head_dim, p->layer, p, err));
            // attention.rs:51-59
            if (p->layer >= p->layers) FAIL("layer out of range");
            if (p->past_len + p->seq > p->max_seq) FAIL("past_len + seq exceeds max_seq");
            return true;
        }
        case SL_OP_SPLIT_HEADS: {
            TRY(input(0, &in0));
            TRY(output(&out));
            p->heads = op.heads;
            p->head_dim = op.head_dim;
            // split_geometry (device.rs:1430-1451)
            if (in0.rank != 3) FAIL("split_heads input shape must be [batch, seq, heads * head_dim]");
            p->batch = in0.e[0];
            p->seq = in0.e[1];
            uint64_t width;
            TRY(checked_mul(p->heads, p->head_dim, &width, err));
            if (in0.e[2] != width) FAIL("split_heads input width must equal heads * head_dim");
            if (out.rank != 4 || out.e[0] != p->batch || out.e[1] != p->heads || out.e[2] != p->seq ||
                out.e[3] != p->head_dim)
                FAIL("split_heads output shape must be [batch, heads, seq, head_dim]");
            return true;
        }
        case SL_OP_MERGE_HEADS: {
            TRY(input(0, &in0));
            TRY(output(&out));
            p->heads = op.heads;
            p->head_dim = op.head_dim;
            if (in0.rank != 4) FAIL("merge_heads input shape must be [batch, heads, seq, head_dim]");
            p->batch = in0.e[0];
            p->seq = in0.e[2];
            if (in0.e[1] != p->heads || in0.e[3] != p->head_dim)
                FAIL("merge_heads input does not match its heads/head_dim attributes");
            uint64_t width;
            TRY(checked_mul(p->heads, p->head_dim, &width, err));
            if (out.rank != 3 || out.e[0] != p->batch || out.e[1] != p->seq || out.e[2] != width)
                FAIL("merge_heads output shape must be [batch, seq, heads * head_dim]");
            return true;
        }
        case SL_OP_CAUSAL_ATTENTION: {
            Dims q, k, v;
            TRY(input(0, &q));
            TRY(input(1, &k));
            TRY(input(2, &v));
            TRY(output(&out));
            TRY(scalar_at(scalars, n_scalars, 0, &p->past_len, err));
            p->layer = op.layer;
            p->heads = op.heads;
            p->kv_heads = op.kv_heads;
            p->head_dim = op.head_dim;
            p->scale = op.scale;
            if (q.rank != 4 || k.rank != 4 || v.rank != 4 || out.rank != 4)
                FAIL("causal_attention operands must have rank 4");
            p->batch = q.e[0];
            p->seq = q.e[2];
            if (q.e[1] != p->heads || q.e[3] != p->head_dim)
                FAIL("causal_attention query shape does not match its attributes");
            if (k.e[0] != p->batch || v.e[0] != p->batch || k.e[1] != p->kv_heads ||
                v.e[1] != p->kv_heads || k.e[2] != p->seq || v.e[2] != p->seq ||
                k.e[3] != p->head_dim || v.e[3] != p->head_dim)
                FAIL("causal_attention key/value shapes must be [batch, kv_heads, seq, head_dim]");
            if (!out.same_as(q)) FAIL("causal_attention output shape must match the query shape");
            if (p->state_index < 0) FAIL("causal_attention requires a State input");
            Dims st;
            TRY(dims_of(iv[p->state_index], &st, err));
            TRY(check_state_geometry(st, p->batch, p->kv_heads, p->head_dim, p->layer, p, err));
            // attention.rs:146-156, then kv_append's checks (attention.rs:51-59)
            if (p->kv_heads == 0) FAIL("kv_heads must be nonzero");
            if (p->heads == 0) FAIL("heads must be nonzero");
            if (p->heads % p->kv_heads != 0) FAIL("heads must be a multiple of kv_heads");
            if (p->layer >= p->layers) FAIL("layer out of range");
            if (p->past_len + p->seq > p->max_seq) FAIL("past_len + seq exceeds max_seq");
            return true;
        }
        case SL_OP_SWIGLU: {
            TRY(only_quantized_at(p->quant, n_in, 0xEu, err));
            TRY(input(0, &in0));
            TRY(input(1, &in1));
            TRY(input(2, &in2));
            TRY(input(3, &in3));
            TRY(output(&out));
            TRY(row_geometry(in0, &p->rows, &p->hidden, err));
            if (in1.rank != 2 || in2.rank != 2 || in3.rank != 2) FAIL("swiglu weights must have rank 2");
            p->inter = in1.e[0];
            if (in1.e[1] != p->hidden || in2.e[0] != p->inter || in2.e[1] != p->hidden ||
                in3.e[0] != p->hidden || in3.e[1] != p->inter)
                FAIL("swiglu weight shapes must be [inter, hidden], [inter, hidden], [hidden, inter]");
            if (!in0.same_as(out)) FAIL("swiglu output shape must match its input");
            // swiglu.rs:50-59
            if (p->hidden == 0) FAIL("swiglu requires a nonzero hidden size");
            if (p->inter == 0) FAIL("swiglu requires a nonzero inter size");
            TRY(quant_matches(p->quant[1], p->inter, p->hidden, err));
            TRY(quant_matches(p->quant[2], p->inter, p->hidden, err));
            return quant_matches(p->quant[3], p->hidden, p->inter, err);
        }
        case SL_OP_RMS_NORM_MATMUL: {
            TRY(only_quantized_at(p->quant, n_in, 0x4u, err));
            TRY(input(0, &in0));
            TRY(input(1, &in1));
            TRY(input(2, &in2));
            TRY(output(&out));
            TRY(row_geometry(in0, &p->rows, &p->hidden, err));
            if (in1.rank != 1 || in1.e[0] != p->hidden) FAIL("rms_norm_matmul weight shape must be [hidden]");
            if (in2.rank != 2 || in2.e[1] != p->hidden)
                FAIL("rms_norm_matmul matrix shape must be [out_features, hidden]");
            p->out_features = in2.e[0];
            if (out.rank != in0.rank) FAIL("rms_norm_matmul output rank must match its input rank");
            for (size_t i = 0; i + 1 < in0.rank; ++i)
                if (out.e[i] != in0.e[i]) FAIL("rms_norm_matmul output prefix must match its input");
            uint64_t width;
            TRY(out.last(&width, err));
            if (width != p->out_features) FAIL("rms_norm_matmul output width must equal out_features");
            // fused.rs:52-61
            if (p->hidden == 0) FAIL("rms_norm_matmul requires a nonzero hidden size");
            if (p->out_features == 0) FAIL("rms_norm_matmul requires a nonzero out_features");
            p->eps = op.eps;
            return quant_matches(p->quant[2], p->out_features, p->hidden, err);
        }
        default:
            *err = Error::unsupported_op(op.code);
            return false;
    }
}

}  // namespace

uint64_t quant_payload_words(uint32_t format, uint64_t n, uint64_t k) {
    uint64_t bytes = format == SL_QFORMAT_INT4 ? n * ((k + 1) / 2) : n * k;
    return (bytes + 3) / 4;
}

bool validate_dispatch(const BufferView& buffers, const sl_op& op, const sl_buffer_ref* inputs,
                       const sl_value* input_values, size_t n_inputs, const sl_buffer_ref* outputs,
                       const sl_value* output_values, size_t n_outputs, const uint32_t* scalars,
                       size_t n_scalars, Plan* plan, Error* err) {
    *plan = Plan();
    plan->code = op.code;
    // The C ABI can carry opcodes sl-ir does not define: the catch-all arm
    // every backend needs (ARCH-0004 §12 item 4).
    if (op.code >= kOpCount) {
        *err = Error::unsupported_op(op.code);
        return false;
    }
    TRY(validate_call(op, input_values, n_inputs, n_outputs, n_scalars, err));
    for (size_t i = 0; i < n_inputs; ++i)
        TRY(validate_port(buffers, inputs[i], input_values[i], false, &plan->quant[i], err));
    QuantOperand unused;
    for (size_t i = 0; i < n_outputs; ++i)
        TRY(validate_port(buffers, outputs[i], output_values[i], true, &unused, err));
    TRY(check_disjoint(inputs, n_inputs, outputs, n_outputs, err));
    for (size_t i = 0; i < n_inputs; ++i)
        if (input_values[i].role == SL_ROLE_STATE) plan->state_index = static_cast<int>(i);
    return op_geometry(op, input_values, n_inputs, output_values, n_outputs, scalars, n_scalars, plan, err);
}

}  // namespace slhip

namespace {

struct TableView : slhip::BufferView {
    const sl_buffer_desc* table;
    size_t n;
    size_t count() const override { return n; }
    const sl_buffer_desc* get(uint32_t id) const override {
        if (id >= n || table[id].kind == SL_BUFFER_NONE) return nullptr;
        return &table[id];
    }
};

}  // namespace

extern "C" sl_status sl_hip_validate_dispatch(const sl_buffer_desc* buffers, size_t n_buffers,
                                              const sl_op* op, const sl_buffer_ref* inputs,
                                              const sl_value* input_values, size_t n_inputs,
                                              const sl_buffer_ref* outputs, const sl_value* output_values,
                                              size_t n_outputs, const uint32_t* scalars, size_t n_scalars,
                                              sl_error* err) {
    TableView view;
    view.table = buffers;
    view.n = n_buffers;
    slhip::Plan plan;
    slhip::Error e;
    if (n_inputs != 0 && input_values == nullptr) e = slhip::Error::execution("inputs and input_values have different lengths");
    else if (n_outputs != 0 && output_values == nullptr) e = slhip::Error::execution("outputs and output_values have different lengths");
    else slhip::validate_dispatch(view, *op, inputs, input_values, n_inputs, outputs, output_values, n_outputs,
                                  scalars, n_scalars, &plan, &e);
    if (err) {
        err->status = e.status;
        err->buffer = e.buffer;
        err->offset = e.offset;
        err->len = e.len;
        err->requested = e.requested;
        err->op = e.op;
        err->reserved = 0;
        err->message = e.message;
    }
    return e.status;
}
