"""Python reader of the .cfmtx text format.

Same surface as code_gen/ss_format/read_compressed_format.py of the
reference (CompressedMatrix, read_compressed_matrix); values are parsed as
Python floats (double), pattern lines keyed by their printed id.
"""


class CompressedMatrix:
    def __init__(self, patterns, num_row, num_col, kernel_rows, kernel_cols):
        self.padded_values_data_array = [[] for _ in range(len(patterns))]
        self.indices_array = [[] for _ in range(len(patterns))]
        self.patterns = patterns
        self.row_panels_pointer = [[] for _ in range(len(patterns))]
        self.num_row = num_row
        self.num_col = num_col
        self.kernel_rows = kernel_rows
        self.kernel_cols = kernel_cols

    def __repr__(self):
        return (f"CompressedMatrix(num_row={self.num_row}, num_col={self.num_col}, "
                f"kernel_rows={self.kernel_rows}, kernel_cols={self.kernel_cols}, "
                f"patterns={self.patterns})")


def read_compressed_matrix(file_path):
    """Header, P pattern lines, then RPP / indices / values lines per pattern."""
    with open(file_path) as f:
        num_row, num_col, kernel_rows, num_patterns, kernel_cols = map(int, f.readline().split())
        patterns = {}
        for _ in range(num_patterns):
            bits, pid = f.readline().split()
            patterns[int(pid)] = bits
        mat = CompressedMatrix(patterns, num_row, num_col, kernel_rows, kernel_cols)
        for i in range(num_patterns):
            mat.row_panels_pointer[i] = [int(t) for t in f.readline().split()]
            mat.indices_array[i] = [int(t) for t in f.readline().split()]
            mat.padded_values_data_array[i] = [float(t) for t in f.readline().split()]
    return mat
