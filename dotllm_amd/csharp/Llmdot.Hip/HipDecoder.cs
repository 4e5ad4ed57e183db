using System.Runtime.CompilerServices;
using System.Text;
using Llmdot.Hip.Native;
using Llmdot.Inference;
using Llmdot.Loading;
using Llmdot.Models;
using Llmdot.Tensors;

namespace Llmdot.Hip;

/// <summary>Options of the device-resident decoder.</summary>
public sealed class HipDecoderOptions
{
    /// <summary>fp16 KV cache (default; half the attention traffic).  False stores fp32 as KvCache does (KV:3-43).</summary>
    public bool KvFp16 { get; init; } = true;

    /// <summary>KV capacity in positions; null: TransformerConfig.ContextLength, as the reference's KvCache.</summary>
    public int? ContextLength { get; init; }

    /// <summary>Tokens per device round trip while streaming (1: every token as soon as it exists).</summary>
    public int ChunkTokens { get; init; } = 1;
}

/// <summary>
/// The LLaMA-like decode loop of InferenceEngine (Generate IE:74-132,
/// ProcessToken IE:134-146, ProcessLlamaLikeLayer IE:184-196, AttentionForward
/// IE:304-450, FFN IE:452-476, final norm and logits IE:575-602) resident on one
/// MI355X: the weights stay in HBM in their GGUF blocks, the KV cache and every
/// activation live on the device, each step is one replayed HIP graph, and the
/// sampled token is fed back on the device.  Created by
/// <see cref="HipBackend.TryCreateDecoder"/> for InferenceEngine, or directly.
/// </summary>
public sealed unsafe class HipDecoder : IDeviceDecoder
{
    private static int s_next;
    private static readonly string[] LayerTensors =
        ["attn_norm", "attn_q", "attn_k", "attn_v", "attn_qkv", "attn_q_norm", "attn_k_norm", "attn_output", "ffn_norm",
         "ffn_gate", "ffn_up", "ffn_down"];

    private readonly LoadedModel _model;
    private readonly HipBackend _backend;
    private readonly TransformerConfig _cfg;
    private readonly string _prefix;
    private readonly List<string> _keys = [];
    private readonly int _chunk;
    private nint _m;

    public int VocabSize { get; }
    public int ContextLength { get; }

    /// <summary>
    /// Whether the device step covers this model: the LLaMA-like template with
    /// RMSNorm, separate or fused Q/K/V, optional per-head Q/K norms, an optional
    /// sliding window, SwiGLU; no softcaps, post-norms, experts or convolution
    /// layers, one KV head count for every layer, and an embedding scale of 1
    /// (the paths of IE:134-196 and IE:304-476 that the LLaMA, Mistral, Phi-3,
    /// Qwen2 and Qwen3 GGUFs take).
    /// </summary>
    public static bool Supports(LoadedModel model, out string? reason)
    {
        var c = model.Config;
        reason = c.Template != ExecutionTemplate.LlamaLike ? $"template {c.Template}"
            : c.NormType != NormType.RmsNorm ? $"norm {c.NormType}"
            : c.FfnType != FfnType.SwiGLU ? $"FFN {c.FfnType}"
            : c.ExpertCount > 0 ? "mixture of experts"
            : c.HasConvLayers ? "convolution layers"
            : c.HasPostNorm ? "post-norms"
            : c.AttnLogitSoftcap.HasValue || c.FinalLogitSoftcap.HasValue ? "logit softcaps"
            : c.EmbeddingScale != 1f ? "embedding scale"
            : c.HeadCountKvPerLayer.Any(h => h != c.HeadCountKv) ? "per-layer KV head counts"
            : null;
        return reason is null;
    }

    public HipDecoder(LoadedModel model, HipBackend backend, HipDecoderOptions? options = null)
    {
        if (!Supports(model, out var why)) throw new NotSupportedException($"HIP decoder: {why}");
        options ??= new HipDecoderOptions();
        if (options.ChunkTokens < 1) throw new ArgumentOutOfRangeException(nameof(options), "ChunkTokens must be at least 1");
        _model = model;
        _backend = backend;
        _cfg = model.Config;
        _chunk = options.ChunkTokens;
        _prefix = $"hipdec{Interlocked.Increment(ref s_next)}/";
        VocabSize = _cfg.VocabSize;
        ContextLength = options.ContextLength ?? _cfg.ContextLength;
        try
        {
            UploadWeights();
            Create(options.KvFp16);
        }
        catch
        {
            Dispose();
            throw;
        }
    }

    private void UploadWeights()
    {
        var names = new List<string> { "token_embd.weight", "output_norm.weight" };
        if (_model.TryGetTensor("output.weight", out _)) names.Add("output.weight");   // else tied (IE:586-589)
        // fused Q/K/V (IE:321-332): the library takes blk.N.attn_qkv.weight in
        // place of the three projections and reads Q, K, V as its row ranges
        var fused = _cfg.QkvLayout == QkvLayout.Fused;
        for (var l = 0; l < _cfg.LayerCount; l++)
            foreach (var t in LayerTensors)
            {
                if (fused ? t is "attn_q" or "attn_k" or "attn_v" : t == "attn_qkv") continue;
                // optional per layer: ffn_norm (attn_norm stands in, IE:547), the Q/K norms (IE:354-373)
                if (t is "ffn_norm" or "attn_q_norm" or "attn_k_norm" && !_model.TryGetTensor($"blk.{l}.{t}.weight", out _))
                    continue;
                names.Add($"blk.{l}.{t}.weight");
            }
        foreach (var name in names)
        {
            var t = _model.GetTensor(name);
            var rows = t.RowCount > 0 ? t.RowCount : 1;
            var cols = (long)(t.ElementCount / (ulong)rows);
            var bytes = (int)TensorSize.ByteCount(t.ElementType, t.ElementCount);
            _backend.Upload(_prefix + name, t.ElementType, t.Data.Span[..bytes], rows, cols);
            _keys.Add(_prefix + name);
        }
    }

    private void Create(bool kvFp16)
    {
        var c = _cfg;
        var ffn = _model.GetTensor("blk.0.ffn_gate.weight").RowCount;
        var prefix = HipNative.Utf8(_prefix)!;
        fixed (byte* pp = prefix)
        {
            var d = new HipNative.ModelDesc
            {
                Hidden = c.HiddenSize, Layers = c.LayerCount, Heads = c.HeadCount, KvHeads = c.HeadCountKv,
                HeadDim = c.HeadDim, Ffn = ffn, Vocab = c.VocabSize, Context = ContextLength,
                RopeDim = c.RopeDimensionCount, Eps = c.NormEpsilon, RopeBase = c.RopeFreqBase,
                // PrecomputeRopeFrequencies (IE:57-72): only Linear scaling changes the table
                RopeLinearFactor = c.RopeScalingType == RopeScalingType.Linear && c.RopeScalingFactor > 1f ? c.RopeScalingFactor : 1f,
                KvFp16 = kvFp16 ? 1 : 0, Bos = c.BosTokenId, SlidingWindow = c.SlidingWindow, KeyPrefix = pp,
            };
            nint m;
            HipNative.Check(HipNative.llmdot_hip_model_create(_backend.Handle, &d, &m));
            _m = m;
        }
    }

    private nint Model
    {
        get
        {
            ObjectDisposedException.ThrowIf(_m == 0, this);
            return _m;
        }
    }

    /// <summary>ProcessToken (IE:134-146): the logits of <paramref name="token"/> at <paramref name="position"/>.</summary>
    public float[] ProcessToken(int token, int position)
    {
        var logits = new float[VocabSize];
        fixed (float* pl = logits)
            HipNative.Check(HipNative.llmdot_hip_decode_step(Model, token, position, pl, null));
        return logits;
    }

    /// <summary>
    /// The prompt loop of IE:84-88 from <paramref name="position0"/>, as batched
    /// MFMA GEMMs when every projection type has a batched kernel; returns the
    /// last token's logits.  The KV cache ends as the sequential loop leaves it.
    /// </summary>
    public float[] Prefill(ReadOnlySpan<int> tokens, int position0)
    {
        var logits = new float[VocabSize];
        fixed (int* pt = tokens)
        fixed (float* pl = logits)
            HipNative.Check(HipNative.llmdot_hip_prefill(Model, pt, tokens.Length, position0, pl, null));
        return logits;
    }

    /// <summary>KvCache.Reset (KV:40).</summary>
    public void Reset() => HipNative.Check(HipNative.llmdot_hip_model_reset(Model));

    /// <summary>The cached K and V rows (kv_heads x head_dim each) of (layer, position), as fp32.</summary>
    public (float[] K, float[] V) ReadKv(int layer, int position)
    {
        var n = _cfg.HeadCountKv * _cfg.HeadDim;
        var k = new float[n];
        var v = new float[n];
        fixed (float* pk = k)
        fixed (float* pv = v)
            HipNative.Check(HipNative.llmdot_hip_kv_read(Model, layer, position, pk, pv));
        return (k, v);
    }

    /// <summary>
    /// InferenceEngine.Generate (IE:74-132) on the device: resets the cache,
    /// processes the prompt (BOS when empty, IE:90-95), then yields each token as
    /// the device produces it -- greedy when Temperature &lt;= 0, else the device
    /// sampler with the reference's uniform draws (new Random(Seed).NextSingle()
    /// per token when Seed &gt;= 0, Random.Shared otherwise; Sampler.cs:158-170).
    /// Stops after EOS (IE:112-115), at MaxTokens, on a stop sequence in the
    /// decoded text (IE:117-125), or when <paramref name="cancellationToken"/> is
    /// cancelled (checked before every token, IE:103).
    /// </summary>
    public async IAsyncEnumerable<int> Generate(int[] promptTokens, GenerationOptions options,
                                                [EnumeratorCancellation] CancellationToken cancellationToken = default)
    {
        var maxTokens = options.MaxTokens;
        Begin(promptTokens, options.Sampling, maxTokens);
        if (maxTokens <= 0) yield break;
        var stops = options.StopSequences;
        var text = stops is { Length: > 0 } ? new StringBuilder() : null;
        var buf = new int[_chunk];
        while (!cancellationToken.IsCancellationRequested)
        {
            var (got, done, rc) = Next(buf);
            for (var i = 0; i < got; i++)
            {
                if (cancellationToken.IsCancellationRequested) yield break;
                var token = buf[i];
                yield return token;
                if (text is not null)
                {
                    text.Append(_model.Tokenizer.Decode(token));
                    var s = text.ToString();
                    foreach (var stop in stops!)
                        if (s.Contains(stop, StringComparison.Ordinal))
                            yield break;
                }
            }
            HipNative.Check(rc);   // the KV cache's end, after its last tokens (KvCache throws there)
            if (done) yield break;
            await Task.CompletedTask.ConfigureAwait(false);
        }
    }

    private void Begin(int[] promptTokens, Sampling.SamplingOptions sampling, int maxTokens)
    {
        var eos = _cfg.EosTokenId;
        fixed (int* pp = promptTokens)
        {
            if (sampling.Temperature <= 0f || maxTokens <= 0)   // Sampler.cs:26-27
            {
                HipNative.Check(HipNative.llmdot_hip_generate_begin(Model, pp, promptTokens.Length, Math.Max(maxTokens, 0), eos, null, null));
                return;
            }
            var draws = new float[maxTokens];
            if (sampling.Seed >= 0)
            {
                // Sampler.cs:160: a new Random(Seed) per draw, so every token uses the same value
                Array.Fill(draws, new Random(sampling.Seed).NextSingle());
            }
            else
            {
                for (var i = 0; i < draws.Length; i++) draws[i] = Random.Shared.NextSingle();
            }
            var opt = new HipNative.Sampling
            {
                Temperature = sampling.Temperature, TopK = sampling.TopK, TopP = sampling.TopP,
                RepeatPenalty = sampling.RepeatPenalty, RepeatWindow = sampling.RepeatPenaltyWindowSize,
            };
            fixed (float* pd = draws)
                HipNative.Check(HipNative.llmdot_hip_generate_begin(Model, pp, promptTokens.Length, maxTokens, eos, &opt, pd));
        }
    }

    private (int Got, bool Done, int Rc) Next(int[] buf)
    {
        int n, done;
        int rc;
        fixed (int* pb = buf)
            rc = HipNative.llmdot_hip_generate_next(Model, buf.Length, pb, &n, &done, null);
        if (rc != HipNative.Ok && rc != HipNative.ERange) HipNative.Check(rc);
        return (n, done != 0, rc);
    }

    public void Dispose()
    {
        var m = Interlocked.Exchange(ref _m, 0);
        if (m != 0) HipNative.llmdot_hip_model_destroy(m);
        foreach (var key in _keys)
        {
            try { _backend.Release(key); }
            catch (ObjectDisposedException) { }   // the backend went first: the library frees the weights with it
        }
        _keys.Clear();
    }
}
