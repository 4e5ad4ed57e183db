using System.Runtime.CompilerServices;
using System.Runtime.InteropServices;
using Llmdot.Hip.Native;
using Llmdot.Inference;
using Llmdot.Loading;
using Llmdot.Tensors;

namespace Llmdot.Hip;

/// <summary>
/// IComputeBackend (src/Llmdot.Core/Inference/Backends/IComputeBackend.cs:7-29)
/// on one AMD Instinct MI355X through libllmdot_hip.so.
///
/// Op level: every member runs on the device with the reference's arithmetic
/// (bit-exact where the C header says so): those on the LLaMA-like decode path
/// (MatMul, MatMulF32, RmsNorm, both ApplyRoPE overloads, Softmax, Silu,
/// SiluInPlace, both Add overloads, both Scale overloads, Mul,
/// DequantizeToFloat, ArgMax) and those of other model templates (LayerNorm,
/// Gelu, GeluScalar, Softcap, Conv1D); MatMul keeps a weight uploaded once
/// under its weightKey resident in HBM.  Spans are host memory, so each call
/// copies its operands over PCIe: correct and useful for validation, not fast.
///
/// Fast path: <see cref="TryCreateDecoder"/> (IDeviceDecodeBackend) gives
/// InferenceEngine a <see cref="HipDecoder"/> that keeps weights, KV cache and
/// activations in HBM and runs the whole token loop on the device.
/// </summary>
public sealed unsafe class HipBackend : IComputeBackend, IDeviceDecodeBackend
{
    private nint _ctx;
    private readonly HashSet<string> _resident = new(StringComparer.Ordinal);
    private readonly List<HipDecoder> _decoders = [];   // created for engines; disposed with the backend
    private readonly object _lock = new();

    /// <summary>Opens device <paramref name="device"/> (HIP ordinal).</summary>
    public HipBackend(int device = 0)
    {
        nint ctx;
        HipNative.Check(HipNative.llmdot_hip_create(device, &ctx));
        _ctx = ctx;
    }

    /// <summary>True when libllmdot_hip.so loads and sees at least one GPU.</summary>
    public static bool IsAvailable => HipNative.TryDeviceCount(out _);

    internal nint Handle
    {
        get
        {
            ObjectDisposedException.ThrowIf(_ctx == 0, this);
            return _ctx;
        }
    }

    /// <summary>Name, architecture (gfx950), CUs, clock and HBM size of the device.</summary>
    public (string Name, string Arch, int ComputeUnits, int ClockMhz, ulong HbmBytes) DeviceInfo
    {
        get
        {
            HipNative.DeviceInfo info;
            HipNative.Check(HipNative.llmdot_hip_get_device_info(Handle, &info));
            return (Marshal.PtrToStringUTF8((nint)info.Name) ?? "", Marshal.PtrToStringUTF8((nint)info.Arch) ?? "",
                    info.ComputeUnits, info.ClockMhz, info.HbmBytes);
        }
    }

    // ---- ICB:9-10 matrix products --------------------------------------------------

    public void MatMul(ReadOnlySpan<float> a, ReadOnlySpan<byte> b, Span<float> result, GgmlType bType, int aCols, int bCols, string? weightKey = null)
    {
        if (aCols <= 0 || bCols <= 0 || result.Length % bCols != 0)
            throw new ArgumentException("result length must be a multiple of bCols");
        var aRows = result.Length / bCols;
        if (a.Length < (long)aRows * aCols) throw new ArgumentException("a is shorter than aRows * aCols");
        var resident = weightKey is not null && IsResident(weightKey);
        var need = (long)bCols * (long)TensorSize.ByteCount(bType, (ulong)aCols);
        if (!resident && b.Length < need) throw new ArgumentException("b is shorter than bCols rows of aCols elements");
        var key = HipNative.Utf8(weightKey);
        fixed (float* pa = a)
        fixed (byte* pb = b)
        fixed (float* pr = result)
        fixed (byte* pk = key)
            HipNative.Check(HipNative.llmdot_hip_matmul(Handle, pa, resident ? null : pb, pr, result.Length, (uint)bType, aCols, bCols, pk));
        if (weightKey is not null) MarkResident(weightKey);
    }

    public void MatMulF32(ReadOnlySpan<float> a, ReadOnlySpan<float> b, Span<float> result, int aCols, int bCols, string? weightKey = null)
    {
        if (aCols <= 0 || bCols <= 0 || result.Length % bCols != 0)
            throw new ArgumentException("result length must be a multiple of bCols");
        var aRows = result.Length / bCols;
        if (a.Length < (long)aRows * aCols) throw new ArgumentException("a is shorter than aRows * aCols");
        var resident = weightKey is not null && IsResident(weightKey);
        if (!resident && b.Length < (long)aCols * bCols) throw new ArgumentException("b is shorter than bCols * aCols");
        var key = HipNative.Utf8(weightKey);
        fixed (float* pa = a)
        fixed (float* pb = b)
        fixed (float* pr = result)
        fixed (byte* pk = key)
            HipNative.Check(HipNative.llmdot_hip_matmul_f32(Handle, pa, resident ? null : pb, pr, result.Length, aCols, bCols, pk));
        if (weightKey is not null) MarkResident(weightKey);
    }

    // ---- ICB:11-12 norms ---------------------------------------------------------------

    public void RmsNorm(ReadOnlySpan<float> input, ReadOnlySpan<float> weights, Span<float> output, float epsilon)
    {
        var n = input.Length;
        if (n == 0) return;
        if (weights.Length < n || output.Length < n) throw new ArgumentException("weights and output must hold input.Length values");
        fixed (float* pi = input)
        fixed (float* pw = weights)
        fixed (float* po = output)
            HipNative.Check(HipNative.llmdot_hip_rms_norm(Handle, pi, pw, po, n, epsilon));
    }

    public void LayerNorm(ReadOnlySpan<float> input, ReadOnlySpan<float> weights, ReadOnlySpan<float> bias, Span<float> output, float epsilon)
    {
        var n = input.Length;
        if (n == 0) return;
        if (weights.Length < n || output.Length < n) throw new ArgumentException("weights and output must hold input.Length values");
        if (bias.Length > 0 && bias.Length < n) throw new ArgumentException("bias must be empty or hold input.Length values");
        fixed (float* pi = input)
        fixed (float* pw = weights)
        fixed (float* pb = bias)
        fixed (float* po = output)
            HipNative.Check(HipNative.llmdot_hip_layer_norm(Handle, pi, pw, bias.Length > 0 ? pb : null, po, n, epsilon));
    }

    // ---- ICB:13-14 rotary embedding (one head of query and key) --------------------------

    public void ApplyRoPE(Span<float> query, Span<float> key, int headDim, int position, float freqBase, int rotaryDim)
    {
        var same = SameSpan(query, key);
        CheckHead(query, key, headDim, same);
        fixed (float* pq = query)
        fixed (float* pk = key)
            HipNative.Check(HipNative.llmdot_hip_apply_rope_base(Handle, pq, same ? pq : pk, headDim, position, freqBase, rotaryDim, same ? 1 : 0));
    }

    public void ApplyRoPE(Span<float> query, Span<float> key, int headDim, int position, ReadOnlySpan<float> freqTable)
    {
        var same = SameSpan(query, key);
        CheckHead(query, key, headDim, same);
        if (2 * freqTable.Length > headDim) throw new ArgumentException("frequency table longer than headDim / 2");
        fixed (float* pq = query)
        fixed (float* pk = key)
        fixed (float* pf = freqTable)
            HipNative.Check(HipNative.llmdot_hip_apply_rope(Handle, pq, same ? pq : pk, headDim, position, pf, freqTable.Length, same ? 1 : 0));
    }

    // ---- ICB:15-19 activations -------------------------------------------------------------

    public void Softmax(Span<float> input, float? softcap = null)
    {
        if (input.IsEmpty) return;
        fixed (float* p = input)
            HipNative.Check(HipNative.llmdot_hip_softmax(Handle, p, input.Length, softcap.HasValue ? 1 : 0, softcap ?? 0f));
    }

    public void Silu(ReadOnlySpan<float> input, Span<float> result)
    {
        if (input.IsEmpty) return;
        if (result.Length < input.Length) throw new ArgumentException("result shorter than input");
        fixed (float* pi = input)
        fixed (float* pr = result)
            HipNative.Check(HipNative.llmdot_hip_silu(Handle, pi, pr, input.Length));
    }

    public void SiluInPlace(Span<float> input)
    {
        if (input.IsEmpty) return;
        fixed (float* p = input)
            HipNative.Check(HipNative.llmdot_hip_silu(Handle, p, p, input.Length));
    }

    public void Gelu(ReadOnlySpan<float> input, Span<float> result)
    {
        if (input.IsEmpty) return;
        if (result.Length < input.Length) throw new ArgumentException("result shorter than input");
        fixed (float* pi = input)
        fixed (float* pr = result)
            HipNative.Check(HipNative.llmdot_hip_gelu(Handle, pi, pr, input.Length));
    }

    /// <summary>VectorMath.Gelu(float): the one-element Gelu, which takes the scalar form.</summary>
    public float GeluScalar(float x)
    {
        float r;
        HipNative.Check(HipNative.llmdot_hip_gelu(Handle, &x, &r, 1));
        return r;
    }

    // ---- ICB:20-24 elementwise ------------------------------------------------------------

    public void Add(Span<float> a, ReadOnlySpan<float> b)
    {
        if (a.IsEmpty) return;
        if (b.Length < a.Length) throw new ArgumentException("b shorter than a");
        fixed (float* pa = a)
        fixed (float* pb = b)
            HipNative.Check(HipNative.llmdot_hip_add(Handle, pa, pb, pa, a.Length));
    }

    public void Add(ReadOnlySpan<float> a, ReadOnlySpan<float> b, Span<float> result)
    {
        if (a.IsEmpty) return;
        if (b.Length < a.Length || result.Length < a.Length) throw new ArgumentException("b and result must hold a.Length values");
        fixed (float* pa = a)
        fixed (float* pb = b)
        fixed (float* pr = result)
            HipNative.Check(HipNative.llmdot_hip_add(Handle, pa, pb, pr, a.Length));
    }

    public void Scale(ReadOnlySpan<float> input, float scale, Span<float> result)
    {
        if (input.IsEmpty) return;
        if (result.Length < input.Length) throw new ArgumentException("result shorter than input");
        fixed (float* pi = input)
        fixed (float* pr = result)
            HipNative.Check(HipNative.llmdot_hip_scale(Handle, pi, scale, pr, input.Length));
    }

    public void Scale(Span<float> input, float scale)
    {
        if (input.IsEmpty) return;
        fixed (float* p = input)
            HipNative.Check(HipNative.llmdot_hip_scale(Handle, p, scale, p, input.Length));
    }

    public void Mul(ReadOnlySpan<float> a, ReadOnlySpan<float> b, Span<float> result)
    {
        if (a.IsEmpty) return;
        if (b.Length < a.Length || result.Length < a.Length) throw new ArgumentException("b and result must hold a.Length values");
        fixed (float* pa = a)
        fixed (float* pb = b)
        fixed (float* pr = result)
            HipNative.Check(HipNative.llmdot_hip_mul(Handle, pa, pb, pr, a.Length));
    }

    // ---- ICB:25-26 other templates' operators -------------------------------------------

    public void Softcap(Span<float> input, float cap)
    {
        if (input.IsEmpty) return;
        fixed (float* p = input)
            HipNative.Check(HipNative.llmdot_hip_softcap(Handle, p, input.Length, cap));
    }

    public void Conv1D(ReadOnlySpan<float> input, ReadOnlySpan<float> weights, Span<float> output, int kernelSize, int inputDim)
    {
        if (inputDim == 0) return;
        var need = (long)kernelSize * inputDim;
        if (input.Length < need || weights.Length < need || output.Length < inputDim)
            throw new IndexOutOfRangeException("input and weights must hold kernelSize * inputDim values, output inputDim");
        fixed (float* pi = input)
        fixed (float* pw = weights)
        fixed (float* po = output)
            HipNative.Check(HipNative.llmdot_hip_conv1d(Handle, pi, pw, po, kernelSize, inputDim));
    }

    // ---- ICB:27-28 ------------------------------------------------------------------------------

    public void DequantizeToFloat(ReadOnlySpan<byte> src, Span<float> dst, GgmlType type, int numRows, int rowElements)
    {
        if (numRows < 0 || rowElements <= 0) throw new ArgumentException("bad DequantizeToFloat shape");
        if (numRows == 0) return;
        var need = (long)numRows * (long)TensorSize.ByteCount(type, (ulong)rowElements);
        if (src.Length < need) throw new ArgumentException("src shorter than numRows rows of rowElements");
        if (dst.Length < (long)numRows * rowElements) throw new ArgumentException("dst shorter than numRows * rowElements");
        fixed (byte* ps = src)
        fixed (float* pd = dst)
            HipNative.Check(HipNative.llmdot_hip_dequantize(Handle, ps, pd, (uint)type, numRows, rowElements));
    }

    public int ArgMax(ReadOnlySpan<float> input)
    {
        if (input.IsEmpty) throw new IndexOutOfRangeException();   // VectorMath.ArgMax reads input[0] (VM:414)
        int index;
        fixed (float* p = input)
            HipNative.Check(HipNative.llmdot_hip_argmax(Handle, p, input.Length, &index));
        return index;
    }

    // ---- the device-resident fast path ------------------------------------------------------

    /// <summary>
    /// A <see cref="HipDecoder"/> for <paramref name="model"/> when the decode
    /// step supports its template (see <see cref="HipDecoder.Supports"/>), else
    /// null: the engine then runs the reference loop over this backend's ops.
    /// </summary>
    public IDeviceDecoder? TryCreateDecoder(LoadedModel model)
    {
        if (!HipDecoder.Supports(model, out _)) return null;
        HipDecoder d;
        try
        {
            d = new HipDecoder(model, this);
        }
        catch (NotSupportedException)
        {
            // a shape the step refuses at creation (e.g. a sliding window with
            // a context beyond the one-launch attention's 16384 positions)
            return null;
        }
        lock (_lock) _decoders.Add(d);
        return d;
    }

    // ---- weights resident under a key ----------------------------------------------------------

    internal bool IsResident(string key)
    {
        lock (_lock)
        {
            if (_resident.Contains(key)) return true;
        }
        var k = HipNative.Utf8(key);
        int present;
        fixed (byte* pk = k)
            HipNative.Check(HipNative.llmdot_hip_has_weight(Handle, pk, &present));
        if (present != 0) MarkResident(key);
        return present != 0;
    }

    internal void MarkResident(string key)
    {
        lock (_lock) _resident.Add(key);
    }

    internal void Upload(string key, GgmlType type, ReadOnlySpan<byte> bytes, long rows, long cols)
    {
        var k = HipNative.Utf8(key);
        fixed (byte* pk = k)
        fixed (byte* pb = bytes)
            HipNative.Check(HipNative.llmdot_hip_upload_weight(Handle, pk, (uint)type, pb, (nuint)bytes.Length, rows, cols));
        MarkResident(key);
    }

    internal void Release(string key)
    {
        var k = HipNative.Utf8(key);
        fixed (byte* pk = k)
            HipNative.Check(HipNative.llmdot_hip_release_weight(Handle, pk));
        lock (_lock) _resident.Remove(key);
    }

    public void Dispose()
    {
        HipDecoder[] decoders;
        lock (_lock)
        {
            decoders = [.. _decoders];
            _decoders.Clear();
        }
        foreach (var d in decoders) d.Dispose();
        var ctx = Interlocked.Exchange(ref _ctx, 0);
        if (ctx != 0) HipNative.llmdot_hip_destroy(ctx);   // deferred by the library while decoders are alive
    }

    private static bool SameSpan(Span<float> a, Span<float> b)
        => Unsafe.AreSame(ref MemoryMarshal.GetReference(a), ref MemoryMarshal.GetReference(b));

    private static void CheckHead(Span<float> query, Span<float> key, int headDim, bool same)
    {
        if (headDim <= 0 || query.Length < headDim || (!same && key.Length < headDim))
            throw new ArgumentException("query and key must hold headDim values");
    }
}
