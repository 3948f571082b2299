"""CPU oracle for the EAGLE3 verify-and-accept path.

TEST INFRASTRUCTURE ONLY. Nothing in the product path (the HIP library, the
host ops under ``neuron-pytorch-native_amd/``) may import, call or link
anything in this package. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only to check or time against it.

Every function restates the reference's algorithm in numpy (float64 unless a
function says otherwise) and cites the reference file:line it follows.

Modules
- ``numerics``  bf16 <-> float32 bit conversions (round-to-nearest-even).
- ``deltanet``  gated-DeltaNet token step, T-token verify, rollback.
- ``gqa``       GQA attention tail (decode and T-token verify), KV append.
- ``fp8``       OCP e4m3fn decode/encode, per-channel quantisation, W8A16 matmul.
- ``accept``    greedy and rejection-sampling acceptance, with the integer
                softmax contract shared bit-for-bit with the HIP kernels.
- ``verify_step`` the 4-layer verify slice composed from the above.

Pinning (what each function is checked against) is listed per module header;
a function with no such check says "parity unpinned" there.
"""
