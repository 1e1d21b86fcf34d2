"""Pattern dictionary of the enumerate-and-sparse-coarsen format.

Drop-in for code_gen/pattern_utiles/pattern_dictionary.py of the reference:
same class, attribute and function names, same ids, same file formats
(including the reference's two dictionary text layouts, which differ:
``export_to_file`` writes ``<id> <bits>`` lines, ``read_pattern_dictionary``
reads a ``m n count`` header then ``<bits> <id>`` lines).

Ids follow the closed form ``id = 2**bits - 1 - int(bit_string, 2)``: id 0 is
the all-ones pattern, id ``2**bits - 2`` has only the last panel row set.
Character ``r`` of a bit string is panel row ``r``.
"""


class PatternTypeDictionary:
    """id <-> bit-string maps (reference: pattern_dictionary.py:1-26)."""

    def __init__(self, m, n):
        self.m = m
        self.n = n
        # attribute names as in the reference (its generators read them)
        self.id_to_patten_bin = {}
        self.pattern_bin_to_id = {}
        self.generated_patterns_ids = []
        self.pattern_id_to_density = {}

    def add_pattern(self, pattern_number, pattern_binary):
        self.id_to_patten_bin[pattern_number] = pattern_binary
        self.pattern_bin_to_id[pattern_binary] = pattern_number

    def append_generated_pattern(self, pattern_number):
        self.generated_patterns_ids.append(pattern_number)

    def is_pattern_generated(self, pattern_number):
        return pattern_number in self.generated_patterns_ids

    def pattern_id_to_number_of_nnz(self, pattern_number):
        return self.id_to_patten_bin[pattern_number].count("1")

    def export_to_file(self, file_path):
        with open(file_path, "w") as f:
            f.writelines(f"{k} {v}\n" for k, v in self.id_to_patten_bin.items())


def _bit_strings(bits):
    top = (1 << bits) - 1
    return [format(top - pid, f"0{bits}b") for pid in range(top)]


def build_patterns_map(kernel_m: int, kernel_n: int) -> dict:
    """tuple(bool) of every non-zero kernel mask -> id, in id order
    (reference: pattern_dictionary.py:29-37)."""
    return {tuple(ch == "1" for ch in s): pid
            for pid, s in enumerate(_bit_strings(kernel_m * kernel_n))}


def generate_pattern_dictionary(m, n=1):
    """PatternTypeDictionary of all non-zero masks (pattern_dictionary.py:40-46)."""
    d = PatternTypeDictionary(m, n)
    for pid, s in enumerate(_bit_strings(m * n)):
        d.add_pattern(pid, s)
    return d


def read_pattern_dictionary(file_path):
    """Header ``m n count``, then ``<bits> <id>`` lines (pattern_dictionary.py:49-60)."""
    with open(file_path) as f:
        m, n, _count = f.readline().split()
        d = PatternTypeDictionary(m, n)
        for line in f:
            bits, key = line.split()
            d.add_pattern(int(key), bits)
    return d
