/*
 * MemoryProvider over HIP device memory (base/code/src/main/java/io/almostrealism/code/
 * MemoryProvider.java:35-199), through HardwareMemoryProvider's reference-queue deallocation
 * (base/hardware/src/main/java/org/almostrealism/hardware/mem/HardwareMemoryProvider.java).
 *
 * Units: like every MemoryProvider, sizes, offsets and lengths are in ELEMENTS of getNumberSize()
 * bytes.  The device computes in fp32, so getNumberSize() is 4 (Precision.FP32.bytes()) and
 *   allocate(int size)                     -> ar_hip_alloc(ctx, size * 4 bytes)
 *   setMem(mem, offset, float[] src, o, n) -> ar_hip_memcpy_h2d(ptr + offset * 4, src + o, n * 4 bytes)
 *   getMem(mem, offset, float[] out, o, n) -> ar_hip_memcpy_d2h(out + o, ptr + offset * 4, n * 4 bytes)
 *   setMem(mem, offset, HipMemory src, so, n) -> ar_hip_memcpy_d2d(ptr + offset * 4, src + so * 4, n * 4 bytes)
 * double[] variants round to float on the way in and widen on the way out, as the reference's
 * fp32 providers do.  Every copy is ordered on the context's stream; host copies return when the
 * data has arrived.
 *
 * Not compiled in this repository (no JDK in the build image).
 */
package org.almostrealism.hardware.hip;

import io.almostrealism.code.Memory;
import org.almostrealism.hardware.HardwareException;
import org.almostrealism.hardware.mem.HardwareMemoryProvider;
import org.almostrealism.hardware.mem.NativeRef;

public class HipMemoryProvider extends HardwareMemoryProvider<HipMemory> {
	private final HipDataContext context;
	private final int numberSize;
	private final long memoryMax;
	private long memoryUsed;

	public HipMemoryProvider(HipDataContext context, int numberSize, long memoryMax) {
		if (numberSize != 4) {
			throw new IllegalArgumentException("HIP device memory holds fp32 values (number size 4), not " + numberSize);
		}
		this.context = context;
		this.numberSize = numberSize;
		this.memoryMax = memoryMax;
	}

	@Override
	public String getName() { return context.getName(); }

	@Override
	public int getNumberSize() { return numberSize; }

	public long getAllocatedMemory() { return memoryUsed; }

	public HipDataContext getContext() { return context; }

	private long ctx() { return context.getHandle(); }

	private long bytes(long elements) { return elements * numberSize; }

	@Override
	public HipMemory allocate(int size) {
		if (size <= 0) throw new IllegalArgumentException("allocation of " + size + " elements");
		long b = bytes(size);
		synchronized (this) {
			if (memoryUsed + b > memoryMax) {
				throw new HardwareException("Memory Max Reached (" + (memoryUsed + b) + " > " + memoryMax + " bytes)");
			}
			memoryUsed += b;
		}
		try {
			return allocated(new HipMemory(this, HIP.alloc(ctx(), b), b));
		} catch (RuntimeException e) {
			synchronized (this) { memoryUsed -= b; }
			throw e;
		}
	}

	@Override
	protected void deallocate(NativeRef<HipMemory> ref) {
		HIP.free(ctx(), ref.getAddress());
		synchronized (this) { memoryUsed -= ref.getSize(); }
	}

	private static void range(HipMemory mem, int offset, int length, long numberSize) {
		if (offset < 0 || length < 0 || (offset + (long) length) * numberSize > mem.getSize()) {
			throw new IllegalArgumentException("range [" + offset + ", " + (offset + (long) length)
					+ ") outside " + mem.getSize() / numberSize + " elements");
		}
	}

	@Override
	public void setMem(HipMemory mem, int offset, float[] source, int srcOffset, int length) {
		range(mem, offset, length, numberSize);
		HIP.setMem(ctx(), mem.getContentPointer(), bytes(offset), source, srcOffset, length);
	}

	@Override
	public void setMem(HipMemory mem, int offset, double[] source, int srcOffset, int length) {
		float[] f = new float[length];
		for (int i = 0; i < length; i++) f[i] = (float) source[srcOffset + i];
		setMem(mem, offset, f, 0, length);
	}

	@Override
	public void setMem(HipMemory mem, int offset, Memory source, int srcOffset, int length) {
		if (source instanceof HipMemory src && src.getProvider() == this) {
			range(mem, offset, length, numberSize);
			range(src, srcOffset, length, numberSize);
			HIP.copy(ctx(), mem.getContentPointer() + bytes(offset), src.getContentPointer() + bytes(srcOffset),
					bytes(length));
		} else {
			setMem(mem, offset, source.toArray(srcOffset, length), 0, length);
		}
	}

	@Override
	public void getMem(HipMemory mem, int sOffset, float[] out, int oOffset, int length) {
		range(mem, sOffset, length, numberSize);
		HIP.getMem(ctx(), mem.getContentPointer(), bytes(sOffset), out, oOffset, length);
	}

	@Override
	public void getMem(HipMemory mem, int sOffset, double[] out, int oOffset, int length) {
		float[] f = new float[length];
		getMem(mem, sOffset, f, 0, length);
		for (int i = 0; i < length; i++) out[oOffset + i] = f[i];
	}
}
