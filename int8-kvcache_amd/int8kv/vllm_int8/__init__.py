"""vLLM integration layer of the INT8 KV cache (counterpart of the reference's vllm_int8/).

Same module names and functions as cjsmt/Int8-kvcache's vllm_int8 package; the operators they
call are this package's HIP kernels.  vLLM itself is imported only inside the functions that
patch it (and at the top of vllm_int8_attention_backend, as in the reference).
"""
