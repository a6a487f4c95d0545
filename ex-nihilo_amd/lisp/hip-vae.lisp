;;;; hip-vae.lisp -- ex-nihilo's VAE decoder and encoder on an AMD MI355X through libexn-hip.so
;;;;
;;;; upload-vae, vae-decode, vae-encode and vae-release of src/cuda-vae.lisp (:15, :94, :138,
;;;; :28) with the same signatures; listed beside hip-dit in ex-nihilo.asd.  Loads after
;;;; hip-dit.lisp, whose shared object, status check and %exn-open it uses.

(in-package #:ex-nihilo)

(sb-alien:define-alien-routine ("exn_vae_create" %exn-vae-create) sb-alien:int
  (ctx sb-sys:system-area-pointer) (out sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_vae_set" %exn-vae-set) sb-alien:int
  (v sb-sys:system-area-pointer) (name sb-alien:c-string) (kind sb-alien:int)
  (data sb-sys:system-area-pointer) (dims sb-sys:system-area-pointer) (ndims sb-alien:int))
(sb-alien:define-alien-routine ("exn_vae_check" %exn-vae-check) sb-alien:int (v sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_vae_decode" %exn-vae-decode) sb-alien:int
  (v sb-sys:system-area-pointer) (latent sb-sys:system-area-pointer) (h sb-alien:int) (w sb-alien:int)
  (rgba sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_vae_check_encoder" %exn-vae-check-encoder) sb-alien:int
  (v sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_vae_encode" %exn-vae-encode) sb-alien:int
  (v sb-sys:system-area-pointer) (rgba sb-sys:system-area-pointer) (h sb-alien:int) (w sb-alien:int)
  (latent sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_vae_release" %exn-vae-release) sb-alien:int (v sb-sys:system-area-pointer))

(defun upload-vae (path &key (device 0))
  "The decoder and encoder in the safetensors at PATH on HIP device DEVICE (the video-only
   time_conv tensors, unused on one frame, stay in the file)."
  (let* ((st (open-vae path))
         (ctx (exn-out-pointer #'%exn-open device))
         (v (exn-out-pointer #'%exn-vae-create ctx)))
    (loop for (name . shape) in (append (vae-expected) (vae-encoder-expected))
          unless (search ".time_conv." name)
            do (let ((f (st-f32 st name))
                     (dims (make-array (length shape) :element-type '(signed-byte 64) :initial-contents shape)))
                 (sb-sys:with-pinned-objects (f dims)
                   (exn-check (%exn-vae-set v name +exn-f32+ (sb-sys:vector-sap f) (sb-sys:vector-sap dims)
                                            (length shape))))))
    (exn-check (%exn-vae-check v))
    (exn-check (%exn-vae-check-encoder v))
    v))

(defun vae-decode (v latent h w)
  "cuda-vae.lisp's vae-decode on the MI355X: the picture (16H x 16W x 4 floats,
   RGBA in -1 .. 1, channels last), its height and its width."
  (let ((px (f32vec (* 16 h 16 w 4))))
    (sb-sys:with-pinned-objects (latent px)
      (exn-check (%exn-vae-decode v (sb-sys:vector-sap latent) h w (sb-sys:vector-sap px))))
    (values px (* 16 h) (* 16 w))))

(defun vae-encode (v px h w)
  "cuda-vae.lisp's vae-encode on the MI355X: PX (H x W x 4 floats, RGBA in -1 .. 1, rows of W
   pixels; H and W multiples of 16) encoded: the latent's mean, 64 x H/16 x W/16 floats
   channel-major, as the decoder takes it (denormalized)."
  (let ((z (f32vec (* 64 (floor h 16) (floor w 16)))))
    (sb-sys:with-pinned-objects (px z)
      (exn-check (%exn-vae-encode v (sb-sys:vector-sap px) h w (sb-sys:vector-sap z))))
    z))

(defun vae-release (v)
  "V's scratch freed (the weights stay)."
  (exn-check (%exn-vae-release v)))
