// DeviceTensor.cs -- a tensor resident in HBM behind the ITensor interface (src/Lokad.Onnx.Tensors/ITensor.cs),
// the device twin of DenseTensor<T> (DenseTensor.cs:31-278): row-major storage, int dims, explicit residency.
// Belongs in src/Lokad.Onnx.Backend.  The HIP provider's operators read and return DeviceTensors; element
// access, printing and enumeration go through a host copy (ToHost), so CPU operators and helpers that expect
// Tensor<T> keep working on ToDenseTensor()'s result.
namespace Lokad.Onnx;

using System;
using System.Collections;
using System.Runtime.InteropServices;

/// <summary>Device storage released to the library's pool when the last handle referring to it is finalised
/// or disposed (lx_tensor_free).</summary>
internal sealed unsafe class DeviceStorage : SafeHandle
{
    private LxTensor t;

    public DeviceStorage(LxTensor owned) : base(IntPtr.Zero, true)
    {
        t = owned;
        SetHandle(owned.Data == IntPtr.Zero ? new IntPtr(-1) : owned.Data);
    }

    public override bool IsInvalid => handle == IntPtr.Zero;

    protected override bool ReleaseHandle()
    {
        fixed (LxTensor* p = &t) return HipNative.lx_tensor_free(p) == 0;
    }
}

public sealed unsafe class DeviceTensor : ITensor, IDisposable
{
    private LxTensor t;                  // a view: dtype, dims, data pointer, capacity (Owns always 0 here)
    private readonly DeviceStorage? storage;   // shared by a tensor and its Reshape aliases; null when borrowed

    private DeviceTensor(LxTensor view, DeviceStorage? storage)
    {
        t = view;
        t.Owns = 0;
        this.storage = storage;
    }

    /// <summary>Takes ownership of an operator's output (Owns = 1: the library allocated it).</summary>
    public static DeviceTensor Own(LxTensor y) => new DeviceTensor(y, y.Owns != 0 ? new DeviceStorage(y) : null);

    /// <summary>A view that borrows its storage from another owner (lx_graph_output, a caller's buffer).</summary>
    public static DeviceTensor Borrow(LxTensor y) => new DeviceTensor(y, null);

    /// <summary>The handle the C ABI takes: a copy of the view (inputs are never written by an operator).</summary>
    internal LxTensor Native => t;

    #region Residency
    /// <summary>The tensor itself if it is already on the device, else an uploaded copy
    /// (DenseTensor buffer -> lx_tensor_alloc + lx_tensor_upload).</summary>
    public static DeviceTensor From(ITensor src) => src as DeviceTensor ?? ToDevice(src);

    public static DeviceTensor ToDevice(ITensor src) => src.ElementType switch
    {
        TensorElementType.Float => Upload((Tensor<float>)src.ToDenseTensor(), src.Name),
        TensorElementType.Double => Upload((Tensor<double>)src.ToDenseTensor(), src.Name),
        TensorElementType.UInt8 => Upload((Tensor<byte>)src.ToDenseTensor(), src.Name),
        TensorElementType.Int8 => Upload((Tensor<sbyte>)src.ToDenseTensor(), src.Name),
        TensorElementType.UInt16 => Upload((Tensor<ushort>)src.ToDenseTensor(), src.Name),
        TensorElementType.Int16 => Upload((Tensor<short>)src.ToDenseTensor(), src.Name),
        TensorElementType.Int32 => Upload((Tensor<int>)src.ToDenseTensor(), src.Name),
        TensorElementType.UInt32 => Upload((Tensor<uint>)src.ToDenseTensor(), src.Name),
        TensorElementType.Int64 => Upload((Tensor<long>)src.ToDenseTensor(), src.Name),
        TensorElementType.UInt64 => Upload((Tensor<ulong>)src.ToDenseTensor(), src.Name),
        TensorElementType.Bool => Upload((Tensor<bool>)src.ToDenseTensor(), src.Name),
        _ => throw new NotSupportedException($"The element type {src.ElementType} has no device storage."),
    };

    static DeviceTensor Upload<T>(Tensor<T> host, string name) where T : unmanaged
    {
        var dense = (DenseTensor<T>)host.ToDenseTensor();
        var dims = new long[Math.Max(dense.Rank, 1)];
        for (int i = 0; i < dense.Rank; i++) dims[i] = dense.Dimensions[i];
        LxTensor y;
        fixed (long* d = dims)
            HipNative.Check(HipNative.lx_tensor_alloc((int)host.ElementType, dense.Rank, d, &y), "lx_tensor_alloc");
        var owned = Own(y);
        using (var pin = dense.Buffer.Pin())
        {
            long nbytes = dense.Length * sizeof(T);
            LxTensor v = owned.t;
            HipNative.Check(HipNative.lx_tensor_upload(&v, pin.Pointer, nbytes), "lx_tensor_upload");
        }
        owned.Name = name;
        return owned;
    }

    /// <summary>A DenseTensor holding the device values (one lx_tensor_download).</summary>
    public ITensor ToHost() => ElementType switch
    {
        TensorElementType.Float => Download<float>(),
        TensorElementType.Double => Download<double>(),
        TensorElementType.UInt8 => Download<byte>(),
        TensorElementType.Int8 => Download<sbyte>(),
        TensorElementType.UInt16 => Download<ushort>(),
        TensorElementType.Int16 => Download<short>(),
        TensorElementType.Int32 => Download<int>(),
        TensorElementType.UInt32 => Download<uint>(),
        TensorElementType.Int64 => Download<long>(),
        TensorElementType.UInt64 => Download<ulong>(),
        TensorElementType.Bool => Download<bool>(),
        _ => throw new NotSupportedException($"The element type {ElementType} has no device storage."),
    };

    DenseTensor<T> Download<T>() where T : unmanaged
    {
        var host = DenseTensor<T>.OfShape(Dims);
        host.Name = Name;
        using var pin = host.Buffer.Pin();
        LxTensor v = t;
        HipNative.Check(HipNative.lx_tensor_download(&v, pin.Pointer, host.Length * sizeof(T)), "lx_tensor_download");
        return host;
    }
    #endregion

    #region ITensor
    public string Name { get; set; } = "";

    public TensorElementType ElementType => (TensorElementType)t.Dtype;

    public Type PrimitiveType => ElementType switch
    {
        TensorElementType.Float => typeof(float),
        TensorElementType.Double => typeof(double),
        TensorElementType.UInt8 => typeof(byte),
        TensorElementType.Int8 => typeof(sbyte),
        TensorElementType.UInt16 => typeof(ushort),
        TensorElementType.Int16 => typeof(short),
        TensorElementType.Int32 => typeof(int),
        TensorElementType.UInt32 => typeof(uint),
        TensorElementType.Int64 => typeof(long),
        TensorElementType.UInt64 => typeof(ulong),
        TensorElementType.Bool => typeof(bool),
        _ => throw new NotSupportedException(),
    };

    public int[] Dims
    {
        get
        {
            var d = new int[t.Rank];
            for (int i = 0; i < t.Rank; i++) d[i] = checked((int)t.Dims[i]);
            return d;
        }
    }

    public int Rank => t.Rank;

    public long Length
    {
        get
        {
            long n = 1;
            for (int i = 0; i < t.Rank; i++) n *= t.Dims[i];
            return n;
        }
    }

    /// <summary>A device copy (Cast to the same element type runs the library's copy kernel).</summary>
    public ITensor Clone()
    {
        LxTensor src = t, y = default;
        HipNative.Check(HipNative.lx_Cast(&src, t.Dtype, &y), "lx_Cast (copy)");
        return Own(y).WithName(Name);
    }

    /// <summary>A zeroed tensor of the same shape, on the host, as DenseTensor.CloneEmpty (DenseTensor.cs:220-223)
    /// gives it: the callers that fill tensors element by element run on the host.</summary>
    public ITensor CloneEmpty() => ToHost().CloneEmpty();

    public ITensor CloneEmpty<U>() where U : unmanaged => ToHost().CloneEmpty<U>();

    /// <summary>DenseTensor.Reshape (DenseTensor.cs:231-242): a view of the same device storage.</summary>
    public ITensor Reshape(params int[] shape)
    {
        var dims = new long[Math.Max(shape.Length, 1)];
        for (int i = 0; i < shape.Length; i++) dims[i] = shape[i];
        LxTensor src = t, y;
        fixed (long* d = dims)
        {
            int st = HipNative.lx_tensor_reshape(&src, shape.Length, d, &y);
            if (st != 0) throw new ArgumentException(HipNative.LastError());
        }
        return new DeviceTensor(y, storage) { Name = Name };
    }

    public ITensor Slice(string indices) => ToHost().Slice(indices);

    public ITensor InsertDim(int dim)
    {
        if (dim >= Rank) throw new IndexOutOfRangeException(nameof(dim));
        var dims = new System.Collections.Generic.List<int>(Dims);
        dims.Insert(dim, 1);
        return Reshape(dims.ToArray());
    }

    public ITensor RemoveDim(int dim)
    {
        if (dim >= Rank) throw new IndexOutOfRangeException(nameof(dim));
        if (Dims[dim] != 1) throw new ArgumentException($"Dimension {dim} is size {Dims[dim]}, not 1.");
        var dims = new System.Collections.Generic.List<int>(Dims);
        dims.RemoveAt(dim);
        return Reshape(dims.ToArray());
    }

    /// <summary>The device operators broadcast by stride-0 reads and need no view; a caller that asks for one
    /// gets the host's BroadcastedTensor.</summary>
    public ITensor BroadcastDim(int dim, int size) => Dims[dim] == size ? this : ToHost().BroadcastDim(dim, size);

    public ITensor ToDenseTensor() => ToHost();

    public Array ToArray() => ToHost().ToArray();

    public object this[params int[] indices]
    {
        get => GetValue(LinearIndex(indices));
        set => SetValue(LinearIndex(indices), value);
    }

    public ITensor this[params object[] indices]
    {
        get => ToHost()[indices];
        set => throw new NotSupportedException("Assigning a slice of a device tensor is not supported; copy it to the host.");
    }

    /// <summary>One element, read from the device (a one-element view at its offset).</summary>
    public object GetValue(int index)
    {
        if (index < 0 || index >= Length) throw new IndexOutOfRangeException();
        var e = HipNative.lx_dtype_size(t.Dtype);
        var buf = stackalloc byte[16];
        LxTensor one;
        HipNative.Check(HipNative.lx_tensor_wrap(t.Dtype, 0, null, t.Data + (nint)(index * e), e, &one), "lx_tensor_wrap");
        HipNative.Check(HipNative.lx_tensor_download(&one, buf, e), "lx_tensor_download");
        return ElementType switch
        {
            TensorElementType.Float => *(float*)buf,
            TensorElementType.Double => *(double*)buf,
            TensorElementType.UInt8 => *buf,
            TensorElementType.Int8 => *(sbyte*)buf,
            TensorElementType.UInt16 => *(ushort*)buf,
            TensorElementType.Int16 => *(short*)buf,
            TensorElementType.Int32 => *(int*)buf,
            TensorElementType.UInt32 => *(uint*)buf,
            TensorElementType.Int64 => *(long*)buf,
            TensorElementType.UInt64 => *(ulong*)buf,
            TensorElementType.Bool => *(bool*)buf,
            _ => throw new NotSupportedException(),
        };
    }

    /// <summary>One element, written to the device.</summary>
    public void SetValue(int index, object value)
    {
        if (index < 0 || index >= Length) throw new IndexOutOfRangeException();
        var e = HipNative.lx_dtype_size(t.Dtype);
        var buf = stackalloc byte[16];
        switch (ElementType)
        {
            case TensorElementType.Float: *(float*)buf = Convert.ToSingle(value); break;
            case TensorElementType.Double: *(double*)buf = Convert.ToDouble(value); break;
            case TensorElementType.UInt8: *buf = Convert.ToByte(value); break;
            case TensorElementType.Int8: *(sbyte*)buf = Convert.ToSByte(value); break;
            case TensorElementType.UInt16: *(ushort*)buf = Convert.ToUInt16(value); break;
            case TensorElementType.Int16: *(short*)buf = Convert.ToInt16(value); break;
            case TensorElementType.Int32: *(int*)buf = Convert.ToInt32(value); break;
            case TensorElementType.UInt32: *(uint*)buf = Convert.ToUInt32(value); break;
            case TensorElementType.Int64: *(long*)buf = Convert.ToInt64(value); break;
            case TensorElementType.UInt64: *(ulong*)buf = Convert.ToUInt64(value); break;
            case TensorElementType.Bool: *(bool*)buf = Convert.ToBoolean(value); break;
            default: throw new NotSupportedException();
        }
        LxTensor one;
        HipNative.Check(HipNative.lx_tensor_wrap(t.Dtype, 0, null, t.Data + (nint)(index * e), e, &one), "lx_tensor_wrap");
        HipNative.Check(HipNative.lx_tensor_upload(&one, buf, e), "lx_tensor_upload");
    }

    /// <summary>Tensor.PrintShape (Tensor.cs:1724).</summary>
    public string PrintShape() => "[" + string.Join(',', Dims) + "]";

    public string PrintData(bool includeWhitespace = true) => ToHost().PrintData(includeWhitespace);

    public IEnumerator GetEnumerator() => ToHost().GetEnumerator();
    #endregion

    int LinearIndex(int[] indices)
    {
        if (indices.Length != Rank) throw new ArgumentException("The number of indices must equal the rank.");
        long k = 0;
        for (int i = 0; i < Rank; i++)
        {
            if (indices[i] < 0 || indices[i] >= t.Dims[i]) throw new IndexOutOfRangeException();
            k = k * t.Dims[i] + indices[i];
        }
        return checked((int)k);
    }

    public DeviceTensor WithName(string name)
    {
        Name = name;
        return this;
    }

    /// <summary>Releases this handle's reference to the storage (the storage itself goes back to the pool when
    /// no alias refers to it any more).</summary>
    public void Dispose() => storage?.Dispose();
}
