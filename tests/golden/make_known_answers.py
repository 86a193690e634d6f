"""Writes known_answers.json: the reference's own known-answer test vectors for
the hot path, transcribed from mpsgraph/gomlx/mpsgraph_test.go (file:line in each
entry).  Values are data (inputs and expected outputs), not code.  Closed forms
the reference computes with math.Exp / math.Sqrt are evaluated here in fp64.

Run:  python tests/golden/make_known_answers.py
"""
import json
import math
import os

e1, e2, e3 = math.exp(1), math.exp(2), math.exp(3)
s3 = math.exp(1.0 / math.sqrt(3.0))
w0, w1 = s3 / (s3 + 1.0), 1.0 / (s3 + 1.0)

CASES = {
    "softmax": {
        "source": "mpsgraph_test.go:1133-1190 (TestFusedSoftmax)",
        "shape": [2, 3], "axis": 1, "tol": 1e-4,
        "x": [1, 2, 3, 1, 1, 1],
        "expected": [e1 / (e1 + e2 + e3), e2 / (e1 + e2 + e3), e3 / (e1 + e2 + e3),
                     1 / 3, 1 / 3, 1 / 3],
    },
    "layernorm_basic": {
        "source": "mpsgraph_test.go:2598-2609 (TestFusedLayerNorm/basic)",
        "shape": [2, 4], "eps": 1e-5, "tol": 1e-3,
        "x": [1, 2, 3, 4, 5, 6, 7, 8],
        "expected": [-1.3416, -0.4472, 0.4472, 1.3416, -1.3416, -0.4472, 0.4472, 1.3416],
    },
    "layernorm_gamma_beta": {
        "source": "mpsgraph_test.go:2611-2623 (TestFusedLayerNorm/with_gamma_beta)",
        "shape": [2, 4], "eps": 1e-5, "tol": 1e-3,
        "x": [1, 2, 3, 4, 5, 6, 7, 8], "gamma": [2, 2, 2, 2], "beta": [1, 1, 1, 1],
        "gamma_shape": [1, 4],
        "expected_first_row": [-1.6833, 0.1056, 1.8944, 3.6833],
    },
    "dot_simple": {
        "source": "mpsgraph_test.go:496-545 (TestDotGeneral/SimpleMatMul)",
        "lhs_shape": [2, 3], "rhs_shape": [3, 2], "lc": [1], "lb": [], "rc": [0], "rb": [],
        "lhs": [1, 2, 3, 4, 5, 6], "rhs": [1, 2, 3, 4, 5, 6], "tol": 1e-4,
        "expected": [22, 28, 49, 64],
    },
    "dot_batched": {
        "source": "mpsgraph_test.go:547-595 (TestDotGeneral/BatchedMatMul)",
        "lhs_shape": [2, 2, 3], "rhs_shape": [2, 3, 2], "lc": [2], "lb": [0], "rc": [1], "rb": [0],
        "lhs": list(range(1, 13)), "rhs": list(range(1, 13)), "tol": 1e-3,
        "expected": [22, 28, 49, 64, 220, 244, 301, 334],
    },
    "dot_bf16": {
        "source": "mpsgraph_test.go:3141-3155 (TestBFloat16/matmul)",
        "lhs_shape": [2, 2], "rhs_shape": [2, 2], "lc": [1], "lb": [], "rc": [0], "rb": [],
        "lhs": [1, 2, 3, 4], "rhs": [5, 6, 7, 8], "tol": 1.0,
        "expected": [19, 22, 43, 50],
    },
    "attention_dot_chain": {
        "source": "mpsgraph_test.go:1638-1724 (TestTransformerBlock)",
        "q": [1, 0, 0, 0, 1, 0], "k": [1, 0, 0, 0, 1, 0], "v": [10, 20, 30, 40, 50, 60],
        "shape": [2, 3], "scale": 1.0 / math.sqrt(3.0), "tol": 1e-3,
        "expected": [w0 * 10 + w1 * 40, w0 * 20 + w1 * 50, w0 * 30 + w1 * 60,
                     w1 * 10 + w0 * 40, w1 * 20 + w0 * 50, w1 * 30 + w0 * 60],
    },
    "sdpa_causal": {
        "source": "mpsgraph_test.go:2996-3015 (TestFusedScaledDotProductAttention/causal_mask)",
        "shape": [1, 1, 3, 2], "scale": 1.0, "causal": True, "tol": 1e-3,
        "q": [1, 0, 0, 1, 1, 1], "k": [1, 0, 0, 1, 1, 1], "v": [1, 0, 0, 1, 0.5, 0.5],
        "expected_first_row": [1, 0],
    },
    "sdpa_bool_mask": {
        "source": "mpsgraph_test.go:3036-3057 (TestFusedScaledDotProductAttention/boolean_mask)",
        "shape": [1, 1, 2, 2], "scale": 1.0, "causal": False, "tol": 1e-3,
        "q": [1, 0, 0, 1], "k": [1, 0, 0, 1], "v": [10, 20, 30, 40],
        "mask": [True, False, True, True],
        "expected_first_row": [10, 20],
    },
    "sdpa_basic_range": {
        "source": "mpsgraph_test.go:2969-2994 (TestFusedScaledDotProductAttention/basic_BHSD)",
        "shape": [1, 1, 2, 2], "scale": 1.0 / math.sqrt(2.0), "causal": False,
        "q": [1, 0, 0, 1], "k": [1, 0, 0, 1], "v": [1, 0, 0, 1],
        "expected_range": [-0.1, 1.1],
    },
    "gather_embedding": {
        "source": "mpsgraph_test.go:599-674 (TestGather/EmbeddingLookup)",
        "table_shape": [4, 3], "table": [10, 11, 12, 20, 21, 22, 30, 31, 32, 40, 41, 42],
        "ids": [1, 3], "expected": [20, 21, 22, 40, 41, 42],
    },
    "argmax": {
        "source": "mpsgraph_test.go:941-991 (TestArgMinMax)",
        "shape": [2, 3], "axis": 1, "x": [1, 5, 3, 8, 2, 6], "expected": [1, 0],
    },
    "iota": {
        "source": "mpsgraph_test.go:785-822 (TestIota)",
        "shape": [2, 3], "axis": 1, "expected": [0, 1, 2, 0, 1, 2],
    },
    "convert_f32_i32": {
        "source": "mpsgraph_test.go:1485-1532 (TestConvertDType)",
        "x": [1.7, 2.3, -0.9], "expected": [1, 2, 0],
    },
    "pad": {
        "source": "mpsgraph_test.go:876-939 (TestPad)",
        "shape": [2, 2], "x": [1, 2, 3, 4], "fill": 0, "start": [1, 0], "end": [0, 1],
        "expected_shape": [3, 3], "expected": [0, 0, 0, 1, 2, 0, 3, 4, 0],
    },
    "dynamic_slice": {
        "source": "mpsgraph_test.go:993-1062 (TestDynamicSlice)",
        "shape": [3, 4], "x": list(range(1, 13)), "starts": [1, 1], "sizes": [2, 2],
        "expected": [6, 7, 10, 11],
    },
    "dynamic_update_slice": {
        "source": "mpsgraph_test.go:1064-1131 (TestDynamicUpdateSlice)",
        "shape": [3, 4], "x": list(range(1, 13)), "update_shape": [2, 2], "update": [100, 200, 300, 400],
        "starts": [1, 1], "expected": [1, 2, 3, 4, 5, 100, 200, 8, 9, 300, 400, 12],
    },
    "scatter_sum": {
        "source": "mpsgraph_test.go:1192-1262 (TestScatterSum)",
        "operand_shape": [4, 2], "operand": [0] * 8, "indices_shape": [3, 1], "indices": [0, 2, 0],
        "updates_shape": [3, 2], "updates": [1, 2, 3, 4, 5, 6],
        "index_vector_axis": 1, "update_window_axes": [1], "inserted_window_axes": [0],
        "scatter_axes_to_operand_axes": [0],
        "expected": [6, 8, 0, 0, 3, 4, 0, 0],
    },
    "sort": {
        "source": "mpsgraph_test.go:3526-3551 (TestSort)",
        "x": [5, 2, 8, 1, 9, 3],
        "ascending": [1, 2, 3, 5, 8, 9], "descending": [9, 8, 5, 3, 2, 1],
    },
    "gelu": {
        "source": "mpsgraph_test.go:2645-2656 (TestFusedGelu)",
        "x": [0.0, 1.0, -1.0, 3.0], "tol": 1e-3,
        "expected": [0.0, 0.8413, -0.1587, 2.9960],
    },
    "dense_no_bias": {
        "source": "mpsgraph_test.go:2809-2825 (TestFusedDense/no_activation_no_bias)",
        "x_shape": [2, 3], "x": [1, 2, 3, 4, 5, 6],
        "w_shape": [3, 4], "w": [1, 0, 0, 0, 0, 1, 0, 0, 0, 0, 1, 0],
        "activation": "none", "tol": 1e-4,
        "expected": [1, 2, 3, 0, 4, 5, 6, 0],
    },
    "dense_bias": {
        "source": "mpsgraph_test.go:2827-2839 (TestFusedDense/with_bias)",
        "x_shape": [2, 2], "x": [1, 0, 0, 1],
        "w_shape": [2, 2], "w": [2, 0, 0, 3], "bias": [10, 20],
        "activation": "none", "tol": 1e-4,
        "expected": [12, 20, 10, 23],
    },
    "dense_relu": {
        "source": "mpsgraph_test.go:2841-2852 (TestFusedDense/relu_activation)",
        "x_shape": [2, 2], "x": [1, -1, -1, 1],
        "w_shape": [2, 2], "w": [1, 0, 0, 1],
        "activation": "relu", "tol": 1e-4,
        "expected": [1, 0, 0, 1],
    },
    "qkv_identity": {
        "source": "mpsgraph_test.go:2900-2931 (TestFusedAttentionQKVProjection/identity_weights)",
        "x_shape": [2, 6], "x": list(range(1, 13)),
        "w_shape": [6, 6], "w": [1.0 if i % 7 == 0 else 0.0 for i in range(36)],
        "query_dim": 2, "key_value_dim": 2, "tol": 1e-4,
        "q": [1, 2, 7, 8], "k": [3, 4, 9, 10], "v": [5, 6, 11, 12],
    },
    "qkv_biases": {
        "source": "mpsgraph_test.go:2933-2962 (TestFusedAttentionQKVProjection/with_biases)",
        "x_shape": [1, 4], "x": [1, 2, 3, 4],
        "w_shape": [4, 6], "w": [1.0 if i in (0, 7, 14, 21) else 0.0 for i in range(24)],
        "bias_q": [10, 20], "bias_k": [100, 200], "bias_v": [1000, 2000],
        "query_dim": 2, "key_value_dim": 2, "tol": 1e-4,
        "q": [11, 22], "k": [103, 204], "v": [1000, 2000],
    },
}

if __name__ == "__main__":
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "known_answers.json")
    with open(out, "w") as f:
        json.dump(CASES, f, indent=1)
    print("wrote", out)
