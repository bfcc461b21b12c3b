"""Host-side behaviour of the intent.jit surface, checked on the CPU (no GPU needed).

Binding rules follow python/intent/runtime/invocation.py:56-159 and
python/intent/runtime/torch_views.py:23-88 of the reference; errors follow its
classes (TypeError for count/type/dtype, ValueError for device/rank/shape/stride/
alias, NotImplementedError for impossible output allocation)."""
import inspect

import pytest
import torch

import intent_amd as intent
import intent_amd.language as I
from intent_amd.examples.kernels.backward.softmax import softmax_backward, softmax_backward_f16
from intent_amd.examples.kernels.contraction.gemm import Activation, bf16_gemm, gemm, gemm_f32, linear_f32
from intent_amd.examples.kernels.normalization.softmax import stable_softmax, stable_softmax_f16
from intent_amd.examples.kernels.sparse.csr_spmv import csr_spmv
from intent_amd.examples.kernels.streaming.attention import (flash_attention_bf16_fwd, flash_attention_fwd,
                                                             flash_gqa_attention_fwd)
from intent_amd.runtime.hip.operators import recognize
from intent_amd.runtime.interface import PublicInterface, StrideSymbol
from intent_amd.runtime.invocation import bind_arguments
from intent_amd.runtime.torch_views import allocate_output, observe_view

CPU = torch.device("cpu")


def bind(defn, args, outputs=None, derived=None, constexprs=None):
    interface = PublicInterface.from_definition(defn, constexprs)
    return bind_arguments(interface, args, outputs,
                          observe_view=lambda p, v: observe_view(p, v, device=CPU),
                          allocate_output=lambda p, s: allocate_output(p, s, device=CPU), derived=derived)


def test_interface_from_definition_matches_reference_schema():
    iface = PublicInterface.from_definition(stable_softmax)
    x, y = iface.parameters
    assert (x.shape, x.dimensions, x.strides, x.noalias, int(x.access)) == ((-1, -1), (1, 2), (None, 1), True, 0)
    assert (y.shape, y.dimensions, int(y.access)) == ((-1, -1), (1, 2), 1)
    static = PublicInterface.from_definition(softmax_backward)
    assert static.parameters[0].shape == (4096, 4097) and static.parameters[0].dimensions == (0, 0)
    attn = PublicInterface.from_definition(flash_attention_fwd, {"CAUSAL": True})
    assert [p.name for p in attn.parameters] == ["q", "k", "v", "output", "scale"]
    assert attn.parameters[1].dimensions[2] != attn.parameters[0].dimensions[2]   # K vs Q
    assert attn.parameters[2].dimensions[:3] == attn.parameters[1].dimensions[:3]
    round_trip = PublicInterface.read(attn.to_json())
    assert round_trip == attn


def test_binding_allocates_and_checks():
    x = torch.zeros(3, 5)
    bound = bind(stable_softmax, (x,))
    (y,) = bound.outputs
    assert y.shape == (3, 5) and y.dtype == torch.float32 and y.is_contiguous()
    with pytest.raises(TypeError):
        bind(stable_softmax, (x.double(),))
    with pytest.raises(ValueError):
        bind(stable_softmax, (torch.zeros(3),))
    with pytest.raises(TypeError):
        bind(stable_softmax, (x, x))
    with pytest.raises(ValueError):                       # strides (None, 1) constraint
        bind(stable_softmax, (torch.zeros(5, 3).t(),))
    with pytest.raises(ValueError):                       # explicit output of the wrong shape
        bind(stable_softmax, (x,), outputs=(torch.zeros(3, 4),))
    with pytest.raises(ValueError):                       # noalias: output aliases the input
        bind(stable_softmax, (x,), outputs=(x,))
    with pytest.raises(ValueError):                       # static extents
        bind(softmax_backward, (torch.zeros(4096, 4096), torch.zeros(4096, 4096)))


def test_shared_dimensions_and_derived_extents():
    a = torch.zeros(4, 6, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        bind(bf16_gemm, (a, torch.zeros(5, 7, dtype=torch.bfloat16)))
    assert bind(bf16_gemm, (a, torch.zeros(6, 7, dtype=torch.bfloat16))).outputs[0].shape == (4, 7)
    iface = PublicInterface.from_definition(csr_spmv)
    with pytest.raises(NotImplementedError):              # R is not derivable from symbols alone
        iface.require_output_allocation()
    ids = {"R1": 1, "NNZ": 2, "C": 3, "R": 4}
    bound = bind(csr_spmv, (torch.zeros(11, dtype=torch.int32), torch.zeros(7, dtype=torch.int32),
                            torch.zeros(7), torch.zeros(9)), derived={ids["R"]: (ids["R1"], -1)})
    assert bound.outputs[0].shape == (10,)
    with pytest.raises(ValueError):
        bind(csr_spmv, (torch.zeros(11, dtype=torch.int32), torch.zeros(7, dtype=torch.int32),
                        torch.zeros(8), torch.zeros(9)), derived={4: (1, -1)})


def test_stride_symbols_bind_consistently():
    @intent.kernel
    def shared(a: I.In[I.f32, ("M", "N"), I.constraints(strides=("S", 1))],
               b: I.Out[I.f32, ("M", "N"), I.constraints(strides=("S", 1))]):
        pass

    iface = PublicInterface.from_definition(shared)
    assert iface.parameters[0].strides == (StrideSymbol("S"), 1)
    big = torch.zeros(4, 10)
    with pytest.raises(ValueError):
        bind(shared, (big[:, :6],), outputs=(torch.zeros(4, 6),))
    bind(shared, (big[:, :6],), outputs=(torch.zeros(4, 10)[:, :6],))


def test_recognition_by_name_and_signature():
    for defn, constexprs in ((stable_softmax, {}), (stable_softmax_f16, {}), (softmax_backward, {}),
                             (softmax_backward_f16, {}), (bf16_gemm, {}), (csr_spmv, {}),
                             (flash_attention_fwd, {"CAUSAL": True}), (gemm_f32, {}), (linear_f32, {}),
                             (gemm, {"ACTIVATION": Activation.RELU}),
                             (flash_gqa_attention_fwd, {"HEAD_GROUP": 4, "CAUSAL": True}),
                             (flash_attention_bf16_fwd, {"HEAD_GROUP": 1, "CAUSAL": False})):
        iface = PublicInterface.from_definition(defn, constexprs)
        assert recognize(defn, iface, tuple(constexprs)).name == defn.__name__

    def f64_softmax(x: I.In[I.f64, ("M", "N")], y: I.Out[I.f64, ("M", "N")]):
        pass

    f64_softmax.__name__ = "stable_softmax"
    impostor = intent.kernel(f64_softmax)
    with pytest.raises(intent.CompilationStageError) as error:
        recognize(impostor, PublicInterface.from_definition(impostor), ())
    assert error.value.stage == "provider_recognition"

    @intent.kernel
    def layer_norm(x: I.In[I.f32, ("M", "N")], y: I.Out[I.f32, ("M", "N")]):
        pass

    with pytest.raises(intent.CompilationStageError):
        recognize(layer_norm, PublicInterface.from_definition(layer_norm), ())


def test_jit_surface_errors_without_gpu():
    with pytest.raises(TypeError):
        intent.jit(lambda x: x, backend="hip")
    with pytest.raises(ValueError):
        intent.jit(stable_softmax, backend="triton")
    kernel = intent.jit(stable_softmax, backend="hip")
    with pytest.raises(ValueError):                       # CPU tensors cannot select a hip device
        kernel.run(torch.zeros(2, 2))
    with pytest.raises(TypeError):
        kernel.prepare(torch.zeros(2, 2), outputs=[torch.zeros(2, 2)])
    with pytest.raises(ValueError):
        kernel.interface                                  # nothing prepared yet
    kernel.close()
    with pytest.raises(intent.LanguageUseError):
        stable_softmax(torch.zeros(1, 1), torch.zeros(1, 1))
    with pytest.raises(intent.LanguageUseError):
        I.exp(1.0)


def test_definitions_keep_reference_signatures():
    """Parameter names, order and annotations of the reference definitions."""
    assert list(inspect.signature(stable_softmax.python_function).parameters) == ["x", "y"]
    assert list(softmax_backward.signature.parameters) == ["probabilities", "upstream", "gradient"]
    assert list(bf16_gemm.signature.parameters) == ["a", "b", "c"]
    assert list(flash_attention_fwd.signature.parameters) == ["q", "k", "v", "output", "scale", "CAUSAL"]
    assert list(csr_spmv.signature.parameters) == ["row_offsets", "column_indices", "values", "vector", "output"]
    assert list(gemm.signature.parameters) == ["a", "b", "c", "ACTIVATION"]
    assert list(gemm_f32.signature.parameters) == ["a", "b", "c"]
    assert list(linear_f32.signature.parameters) == ["x", "weight", "output"]
    for defn in (flash_gqa_attention_fwd, flash_attention_bf16_fwd):
        assert list(defn.signature.parameters) == ["q", "k", "v", "output", "scale", "HEAD_GROUP", "CAUSAL"]
    assert (Activation.NONE.value, Activation.RELU.value) == (0, 1)


def test_sibling_plan_errors_before_launch():
    """Constexpr and head-group checks of the plans fire before the library is touched."""
    from types import SimpleNamespace

    from intent_amd.runtime.hip import operators

    with pytest.raises(intent.CompilationStageError) as error:
        operators._activation_code(7)
    assert error.value.stage == "provider_configuration"
    assert operators._activation_code(Activation.RELU) == 1 and operators._activation_code(0) == 0
    q, k = torch.zeros(1, 6, 4, 128), torch.zeros(1, 4, 4, 128)
    bound = SimpleNamespace(arguments=(q, k, k, q, 1.0))
    plan = operators._attention_grouped(operators.F16)
    with pytest.raises(ValueError):                       # 6 query heads != 4 key heads * 2
        plan(None, bound, {"HEAD_GROUP": 2, "CAUSAL": True}, CPU)
    with pytest.raises(intent.CompilationStageError):
        plan(None, bound, {"HEAD_GROUP": 0, "CAUSAL": True}, CPU)
    with pytest.raises(intent.CompilationStageError):
        plan(None, bound, {"HEAD_GROUP": True, "CAUSAL": True}, CPU)
    iface = PublicInterface.from_definition(flash_gqa_attention_fwd, {"HEAD_GROUP": 2, "CAUSAL": True})
    with pytest.raises(intent.CompilationStageError):     # constexprs in the wrong order are another contract
        recognize(flash_gqa_attention_fwd, iface, ("CAUSAL", "HEAD_GROUP"))


def test_attention_backward_definitions_and_sequence():
    from intent_amd.examples.kernels.backward.attention import (attention_backward_delta, attention_backward_dkdv,
                                                                attention_backward_dq)
    from intent_amd.runtime import PreparedSequence

    options = {"HEAD_GROUP": 4, "CAUSAL": True}
    for defn, constexprs in ((attention_backward_delta, {}), (attention_backward_dkdv, options),
                             (attention_backward_dq, options)):
        iface = PublicInterface.from_definition(defn, constexprs)
        assert recognize(defn, iface, tuple(constexprs)).name == defn.__name__
    assert list(attention_backward_dq.signature.parameters) == [
        "q", "k", "v", "grad_output", "lse", "delta", "grad_q", "scale", "HEAD_GROUP", "CAUSAL"]
    assert list(attention_backward_dkdv.signature.parameters) == [
        "q", "k", "v", "grad_output", "lse", "delta", "grad_k", "grad_v", "scale", "HEAD_GROUP", "CAUSAL"]
    assert PublicInterface.from_definition(attention_backward_dq, options).parameters[6].noalias

    order = []

    class Call:
        def __init__(self, name):
            self.name, self.observation = name, None

        def compile(self):
            order.append(("compile", self.name))

        def launch(self):
            order.append(("launch", self.name))

    sequence = PreparedSequence((Call("a"), PreparedSequence((Call("b"), Call("c")), outputs=None)), outputs=(1, 2))
    sequence.compile()
    sequence.launch()
    assert order == [("compile", "a"), ("compile", "b"), ("compile", "c"), ("launch", "a"), ("launch", "b"),
                     ("launch", "c")]
    assert sequence.result() == (1, 2) and sequence.kernel_count == 3
    with pytest.raises(ValueError):
        PreparedSequence((), outputs=None)


def test_paged_decode_definitions_recognised_with_reference_signatures():
    from intent_amd.examples.kernels.streaming.paged_attention import paged_gqa_decode_partials
    from intent_amd.examples.kernels.streaming.splitk_reduce import splitk_attention_f32_to_f16_reduce
    from intent_amd.examples.programs.composition import PagedDecode

    options = {"PAGE_SIZE": 16, "HEAD_GROUP": 4, "SPLITS": 8}
    iface = PublicInterface.from_definition(paged_gqa_decode_partials, options)
    assert recognize(paged_gqa_decode_partials, iface, tuple(options)).name == "paged_gqa_decode_partials"
    assert list(paged_gqa_decode_partials.signature.parameters) == [
        "q", "key_cache", "value_cache", "page_offsets", "page_indices", "sequence_lengths", "split_offsets",
        "partial_lse", "partial_output", "scale", "PAGE_SIZE", "HEAD_GROUP", "SPLITS"]
    # the SPLITS constexpr sizes both outputs, so they allocate from the inputs alone
    outputs = [p for p in iface.parameters if getattr(p, "writable", False)]
    assert [p.shape[-1] for p in outputs][:1] == [8]
    iface.require_output_allocation()
    merge = PublicInterface.from_definition(splitk_attention_f32_to_f16_reduce, {})
    assert recognize(splitk_attention_f32_to_f16_reduce, merge, ()).name == "splitk_attention_f32_to_f16_reduce"
    assert list(splitk_attention_f32_to_f16_reduce.signature.parameters) == ["partial", "partial_lse", "output"]
    assert PagedDecode.mutable_inputs == ()


@pytest.mark.parametrize("name,options,parameters", [
    ("flash_attention_bias_fwd", {}, ["q", "k", "v", "bias", "output", "scale"]),
    ("mla_prefill", {"HEAD_GROUP": 4}, ["q", "qpe", "k", "kpe", "v", "output", "scale", "HEAD_GROUP"]),
    ("grouped_flash_decode_partials", {"HEAD_GROUP": 4, "P": 8, "SPLIT_SIZE": 1024},
     ["q", "k", "v", "partial_lse", "partial_output", "scale", "HEAD_GROUP", "P", "SPLIT_SIZE"]),
    ("continuous_gqa_decode", {"HEAD_GROUP": 4},
     ["q", "k", "v", "valid_mask", "output", "scale", "HEAD_GROUP"]),
    ("varlen_gqa_decode_with_sink_logits", {"HEAD_GROUP": 4, "MAX_BLOCKS": 64},
     ["q", "k", "v", "cu_seqlens", "sink", "output", "block_logits", "scale", "HEAD_GROUP", "MAX_BLOCKS"]),
])
def test_attention_variants_recognised_with_reference_signatures(name, options, parameters):
    """streaming/attention.py:556-836: the bias and decode definitions keep the reference's
    parameter names and order, and the provider recognises each by name and signature."""
    import intent_amd.examples.kernels.streaming.attention as attention

    definition = getattr(attention, name)
    assert list(definition.signature.parameters) == parameters
    iface = PublicInterface.from_definition(definition, options)
    assert recognize(definition, iface, tuple(options)).name == name


def test_csr_spmm_definition_recognised_with_reference_signature():
    from intent_amd.examples.kernels.sparse.csr_spmm import csr_spmm

    iface = PublicInterface.from_definition(csr_spmm, {})
    assert recognize(csr_spmm, iface, ()).name == "csr_spmm"
    assert list(csr_spmm.signature.parameters) == ["row_offsets", "column_indices", "values", "dense", "output"]


def test_definition_modules_export_the_reference_extents():
    """The reference's examples import the extent constants of the definition modules
    (examples/programs/irregular.py:14-15 imports ROWS, COLUMNS, NONZEROS, NONZEROS_PER_ROW from
    csr_spmv); the same names carry the same values here."""
    import math

    from intent_amd.examples.kernels.contraction import gemm
    from intent_amd.examples.kernels.normalization import softmax
    from intent_amd.examples.kernels.sparse import csr_spmv
    from intent_amd.examples.kernels.streaming import attention

    assert (csr_spmv.ROWS, csr_spmv.COLUMNS, csr_spmv.NONZEROS_PER_ROW) == (32768, 32768, 32)
    assert csr_spmv.NONZEROS == 32768 * 32
    assert (softmax.ROWS, softmax.COLUMNS) == (8192, 8192)
    assert (gemm.M, gemm.K, gemm.N) == (4096, 4096, 14336)
    assert (attention.BATCH, attention.HEADS, attention.SEQUENCE, attention.HEAD_DIMENSION) == (4, 32, 4096, 128)
    assert attention.SCALE == 1.0 / math.sqrt(128)
