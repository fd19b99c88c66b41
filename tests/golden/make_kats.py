"""Writes tests/golden/kats.json: the reference's own known-answer tests for
the dense-contraction path, as data (inputs + expected outputs).

Sources (under /root/reference, read as text):
  tests/unit/test_matmul.cu:13-68          2x2 and diag(1..4)*I GEMMs
  tests/unit/test_tensor.cu:189-248        2x2, 2x3*3x4 partial identity, (0.1 i)*I
  tests/unit/test_tensor_ops.py:211-218    2x2 matmul
  tests/unit/test_autograd.py:85-94        grads of sum(A@B)
  tests/unit/test_nn.py:50-76              Linear with fixed weights / bias
  tests/unit/test_kernels.cu:324-425       conv2d forward identity / 3x3 / bias / pad
  tests/unit/test_advanced_kernels.cu:198-242  conv backward data / weight
  benchmarks/test_mma.cu:40-119            MMA fragment tests (A*I, integer pattern)

Run: python tests/golden/make_kats.py  (no GPU, no reference import).
"""
import json
import os


def mm(a, b):
    return [[sum(a[i][k] * b[k][j] for k in range(len(b))) for j in range(len(b[0]))]
            for i in range(len(a))]


def main():
    kats = {}
    kats["matmul_2x2"] = {"A": [[1, 2], [3, 4]], "B": [[5, 6], [7, 8]],
                          "C": [[19, 22], [43, 50]]}
    kats["matmul_diag_identity"] = {
        "A": [[float(i + 1) if i == j else 0.0 for j in range(4)] for i in range(4)],
        "B": [[1.0 if i == j else 0.0 for j in range(4)] for i in range(4)],
        "C": [[float(i + 1) if i == j else 0.0 for j in range(4)] for i in range(4)]}
    kats["matmul_partial_identity"] = {
        "A": [[1, 2, 3], [4, 5, 6]],
        "B": [[1, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 0]],
        "C_row0": [1, 2, 3, 0]}
    kats["matmul_scaled_identity_8"] = {
        "A": [[0.1 * (i * 8 + j) for j in range(8)] for i in range(8)],
        "atol": 0.01}
    kats["autograd_sum_matmul"] = {"A": [[1, 2], [3, 4]], "B": [[5, 6], [7, 8]],
                                   "dA": [[11, 15], [11, 15]], "dB": [[4, 4], [6, 6]]}
    kats["linear_fixed_weight"] = {"W": [[1, 0, 0], [0, 1, 0]], "b": [0, 0],
                                   "x": [[10, 20, 30], [40, 50, 60]],
                                   "y": [[10, 20], [40, 50]]}
    kats["linear_identity_bias"] = {"W": [[1, 0], [0, 1]], "b": [100, 200],
                                    "x": [[1, 2]], "y": [[101, 202]]}
    kats["conv_identity_1x1"] = {
        "x_shape": [1, 1, 4, 4], "x": [float(i + 1) for i in range(16)],
        "w_shape": [1, 1, 1, 1], "w": [1.0], "bias": [0.0], "stride": [1, 1],
        "padding": [0, 0], "y": [float(i + 1) for i in range(16)]}
    kats["conv_3x3_ones"] = {
        "x_shape": [1, 1, 3, 3], "x": [1.0] * 9, "w_shape": [1, 1, 3, 3],
        "w": [1.0] * 9, "bias": None, "stride": [1, 1], "padding": [0, 0], "y": [9.0]}
    kats["conv_3x3_bias"] = {
        "x_shape": [1, 1, 3, 3], "x": [1.0] * 9, "w_shape": [1, 1, 3, 3],
        "w": [1.0] * 9, "bias": [10.0], "stride": [1, 1], "padding": [0, 0], "y": [19.0]}
    kats["conv_3x3_pad1"] = {
        "x_shape": [1, 1, 3, 3], "x": [1.0] * 9, "w_shape": [1, 1, 3, 3],
        "w": [1.0] * 9, "bias": None, "stride": [1, 1], "padding": [1, 1],
        "y": [4.0, 6.0, 4.0, 6.0, 9.0, 6.0, 4.0, 6.0, 4.0]}
    kats["conv_bwd_data_1x1_w2"] = {
        "dy_shape": [1, 1, 3, 3], "dy": [1.0] * 9, "w_shape": [1, 1, 1, 1], "w": [2.0],
        "x_shape": [1, 1, 3, 3], "stride": [1, 1], "padding": [0, 0], "dx": [2.0] * 9}
    kats["conv_bwd_weight_ones"] = {
        "dy_shape": [1, 1, 3, 3], "dy": [1.0] * 9, "x_shape": [1, 1, 3, 3], "x": [1.0] * 9,
        "w_shape": [1, 1, 1, 1], "stride": [1, 1], "padding": [0, 0], "dw": [9.0]}
    A = [[float(i * 8 + j + 1) for j in range(8)] for i in range(16)]
    I8 = [[1.0 if i == j else 0.0 for j in range(8)] for i in range(8)]
    kats["mma_identity"] = {"A": A, "B": I8, "C": mm(A, I8)}
    hA = [float((i * 3 + 7) % 11) - 5.0 for i in range(128)]
    hB = [float((i * 7 + 3) % 13) - 6.0 for i in range(64)]
    A2 = [hA[r * 8:(r + 1) * 8] for r in range(16)]
    B2 = [hB[r * 8:(r + 1) * 8] for r in range(8)]
    kats["mma_integer_pattern"] = {"A": A2, "B": B2, "C": mm(A2, B2)}
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kats.json")
    with open(out, "w") as f:
        json.dump(kats, f, indent=1)
    print("wrote", out)


if __name__ == "__main__":
    main()
