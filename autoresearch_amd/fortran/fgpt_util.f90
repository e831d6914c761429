! fgpt_util.f90 -- host helpers shared by the ids-in/ids-out harness
! (fgpt_run) and the drop-in check programs under tests/fortran: command-line
! arguments, ids files, the callers' RoPE tables (src/app/chat_text.f90:
! 225-235, src/app/eval_bpb.f90:117-126) and a wall clock.
module fgpt_util
  use, intrinsic :: iso_c_binding
  use, intrinsic :: iso_fortran_env, only: error_unit, int64
  use fgpt_c
  implicit none
  private
  public :: iarg, rarg, sarg, read_ids, rope_tables, set_rope_rows, now, stop_rc

contains

  integer function iarg(i)
    integer, intent(in) :: i
    character(len=64) :: s
    integer :: ios
    call get_command_argument(i, s)
    read (s, *, iostat=ios) iarg
    if (ios /= 0) then
      write (error_unit, '(A,I0,2A)') 'bad integer argument ', i, ': ', trim(s)
      stop 2
    end if
  end function iarg

  real(8) function rarg(i)
    integer, intent(in) :: i
    character(len=64) :: s
    integer :: ios
    call get_command_argument(i, s)
    read (s, *, iostat=ios) rarg
    if (ios /= 0) then
      write (error_unit, '(A,I0,2A)') 'bad real argument ', i, ': ', trim(s)
      stop 2
    end if
  end function rarg

  character(len=512) function sarg(i)
    integer, intent(in) :: i
    call get_command_argument(i, sarg)
  end function sarg

  ! Every whitespace-separated integer of the file, in order (any number per
  ! line).
  subroutine read_ids(path, ids, n)
    character(*), intent(in) :: path
    integer(c_int), allocatable, intent(out) :: ids(:)
    integer, intent(out) :: n
    integer :: u, ios, j, nt
    integer(c_int), allocatable :: tmp(:)
    character(len=65536) :: line
    logical :: intok
    allocate (ids(1024))
    n = 0
    open (newunit=u, file=path, status='old', action='read', iostat=ios)
    if (ios /= 0) then
      write (error_unit, '(2A)') 'cannot open ', trim(path)
      stop 1
    end if
    do
      read (u, '(A)', iostat=ios) line
      if (ios /= 0) exit
      nt = 0
      intok = .false.
      do j = 1, len_trim(line)
        if (line(j:j) == ' ' .or. line(j:j) == char(9) .or. line(j:j) == ',') then
          intok = .false.
        else if (.not. intok) then
          intok = .true.
          nt = nt + 1
        end if
      end do
      if (nt == 0) cycle
      do while (n + nt > size(ids))
        allocate (tmp(2*size(ids)))
        tmp(1:size(ids)) = ids
        call move_alloc(tmp, ids)
      end do
      read (line, *, iostat=ios) ids(n+1:n+nt)
      if (ios /= 0) then
        write (error_unit, '(2A)') 'bad ids line in ', trim(path)
        stop 1
      end if
      n = n + nt
    end do
    close (u)
  end subroutine read_ids

  ! chat_text.f90:225-235 / eval_bpb.f90:117-126
  subroutine rope_tables(ntot, hd, cos_b, sin_b)
    integer, intent(in) :: ntot, hd
    real(c_float), allocatable, intent(out) :: cos_b(:), sin_b(:)
    integer :: i, j
    real(c_float) :: theta, ang
    allocate (cos_b(ntot*(hd/2)), sin_b(ntot*(hd/2)))
    do i = 1, ntot
      do j = 1, hd/2
        theta = 10000.0_c_float ** (-2.0_c_float * real(j-1, c_float) / real(hd, c_float))
        ang = real(i-1, c_float) * theta
        cos_b((i-1)*(hd/2)+j) = cos(ang)
        sin_b((i-1)*(hd/2)+j) = sin(ang)
      end do
    end do
  end subroutine rope_tables

  ! RoPE rows [pos0, pos0+n) of the host tables into the engine (the device
  ! loop reads them without a host round trip per step)
  subroutine set_rope_rows(model, pos0, n, hd, cos_b, sin_b)
    type(c_ptr), intent(in) :: model
    integer(c_int), intent(in) :: pos0
    integer, intent(in) :: n, hd
    real(c_float), intent(in) :: cos_b(:), sin_b(:)
    integer(c_int32_t) :: rc
    if (n < 1) return
    rc = fg_set_rope(model, pos0, n, cos_b(pos0*(hd/2)+1:), sin_b(pos0*(hd/2)+1:))
    if (rc /= FG_OK) then
      write (error_unit, '(2A)') 'fg_set_rope: ', fg_error_message()
      stop 1
    end if
  end subroutine set_rope_rows

  real(8) function now()
    integer(int64) :: c, r
    call system_clock(c, r)
    now = real(c, 8) / real(r, 8)
  end function now

  subroutine stop_rc(what, rc)
    character(*), intent(in) :: what
    integer(c_int32_t), intent(in) :: rc
    write (error_unit, '(4A,I0,A)') what, ': ', fg_error_message(), ' (rc ', rc, ')'
    stop 1
  end subroutine stop_rc

end module fgpt_util
